"""Batch-1 decode through a stack of MoE layers in one kernel launch (lmoe_stack_decode).

The reference decodes a token layer by layer, each layer's router, experts and combine a chain of kernels
(stream_fast.py:4352-4377 over gguf_experts.experts, gguf_experts.py:803-819). Here the whole stack is one
persistent cooperative launch of one workgroup a CU; the layer boundaries, and the three all-to-all hand-offs inside a
layer (x to every expert row, the router logits to every top-k, h to every down row), go through a device workspace
as epoch-tagged words instead of kernel boundaries. Numerics are the decode chain's: f16 activations between
layers, fp32 accumulation, h rounded to f16, the router logits summed in a fixed order that the test oracle restates.

    st = Stack(layers)            # MoELayer objects of one shape, Q4_0 or Q4_K, f16 router weights
    st.step(x, out)               # x, out: [H] (or [1, H]) float16 on the GPU; out = x after every layer
    st.check()                    # synchronises; raises if a launch's internal wait ran out

With ``trace=True`` the stack also keeps, per layer, the MoE output before the residual (``y`` [L, H] f32), the
picked experts (``ids`` [L, k]) and their scores (``scores`` [L, k]); ``layer_inputs()`` and ``logits()`` read
x_l and the router logits of the last step back from the workspace.
"""
import ctypes

import torch

from . import _lib
from ._lib import call, ptr, qcode, stream


class Stack:
    def __init__(self, layers, trace=False, device="cuda"):
        if not layers:
            raise ValueError("a stack needs at least one layer")
        L0 = layers[0]
        t = L0.types[0]
        if any(x != t for x in L0.types) or t not in _lib.Q4_TYPES:
            raise ValueError(f"the fused stack takes one block type, Q4_0 or Q4_K, for every projection, got {L0.types}")
        for L in layers:
            if (L.types, L.E, L.I, L.H, L.k, L.norm, L.Is) != (L0.types, L0.E, L0.I, L0.H, L0.k, L0.norm, L0.Is):
                raise ValueError("every layer of a stack has the first layer's shape, types, top-k and norm")
            if L.wr is None or L.wr.dtype != torch.float16:
                raise ValueError("the fused stack needs float16 router weights")
            if L.shared is not None and (L.wsg is None or L.wsg.dtype != torch.float16):
                raise ValueError("the fused stack needs a float16 shared-expert gate weight")
        self.layers = layers
        self.L, self.H, self.E, self.k, self.I, self.Is = len(layers), L0.H, L0.E, L0.k, L0.I, L0.Is
        self.qtype = qcode(t)
        self.norm = int(L0.norm)

        def table(get):
            return torch.tensor([get(L).data_ptr() for L in layers], dtype=torch.int64, device=device)

        self._tabs = [table(lambda L: L.wg), table(lambda L: L.wu), table(lambda L: L.wd), table(lambda L: L.wr)]
        if self.Is:
            self._tabs += [table(lambda L: L.wsg), table(lambda L: L.shared[0]), table(lambda L: L.shared[1]),
                           table(lambda L: L.shared[2])]
        else:
            self._tabs += [None] * 4
        nbytes = _lib.lib().lmoe_stack_workspace_bytes(self.L, self.H, self.E, self.k, self.I, self.Is)
        if nbytes == 0:
            raise ValueError("lmoe_stack_workspace_bytes refused the shape")
        self.workspace = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        self.y = self.ids = self.scores = None
        if trace:
            self.y = torch.zeros((self.L, self.H), dtype=torch.float32, device=device)
            self.ids = torch.zeros((self.L, self.k), dtype=torch.int32, device=device)
            self.scores = torch.zeros((self.L, self.k), dtype=torch.float32, device=device)
        self._x0 = None

    def nbytes_touched(self, n_unique_per_layer):
        """Algorithmic HBM bytes of one step: each layer's touched experts, shared expert and router weights."""
        return sum(L.nbytes_touched(n) for L, n in zip(self.layers, n_unique_per_layer))

    def step(self, x, out):
        """out = x_L for x_0 = x; x and out are float16 [H] or [1, H] on the GPU (out may not alias x)."""
        if x.dtype != torch.float16 or out.dtype != torch.float16:
            raise ValueError("the fused stack takes and gives float16 activations")
        if x.numel() != self.H or out.numel() != self.H:
            raise ValueError(f"one token of {self.H} values expected")
        if x.data_ptr() == out.data_ptr():
            raise ValueError("out may not alias x")
        tabs = [ptr(t) for t in self._tabs]
        call("lmoe_stack_decode", self.L, self.H, self.E, self.k, self.I, self.Is, self.qtype, self.norm, *tabs,
             ptr(x), ptr(out), ptr(self.workspace), ptr(self.y), ptr(self.ids), ptr(self.scores), stream())
        self._x0 = x
        return out

    def status(self):
        """The workspace's status word (0: every wait ended in time); synchronises the current stream."""
        v = ctypes.c_uint32(0)
        call("lmoe_stack_status", ptr(self.workspace), ctypes.byref(v), stream())
        return int(v.value)

    def check(self):
        """Raise RuntimeError (and clear the workspace, so the stack can run again) if a launch timed out."""
        s = self.status()
        if s:
            self.workspace.zero_()
            raise RuntimeError(f"lmoe_stack_decode: a launch's internal wait ran out (status {s}); workspace cleared")

    def _words(self):
        ws = self.workspace[256:].view(torch.int64)
        L, H = self.L, self.H
        etot = self.E + (1 if self.Is else 0)
        nx = (L - 1) * (H // 2)
        return ws[:nx].view(max(L - 1, 0), H // 2), ws[nx:nx + L * etot].view(L, etot)

    def layer_inputs(self):
        """x_0 .. x_{L-1} of the last step as float16 [L, H] (x_0 is the step's input)."""
        xw, _ = self._words()
        body = (xw & 0xFFFFFFFF).to(torch.int32).view(torch.float16).reshape(self.L - 1, self.H)
        return torch.cat([self._x0.reshape(1, self.H), body], 0)

    def logits(self):
        """The router logits of the last step, float32 [L, E (+1: the shared-expert gate)]."""
        _, lw = self._words()
        return (lw & 0xFFFFFFFF).to(torch.int32).view(torch.float32)
