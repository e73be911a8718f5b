"""Per-workgroup phase timeline of the decode kernels (lmoe_timeline_* in include/larder_moe.h).

While a ``Timeline`` is entered, the router GEMV, the fused gate/up and the two-wavefront down that this thread
launches (also into a graph under capture) run their stamping forms: every workgroup writes the device's
constant-rate wall clock into its row of 8 at each phase it reaches (``PHASES``). The launches give the same results
bit for bit as the unstamped forms. A measurement tool: the reference has no counterpart.
"""
import ctypes

import numpy as np
import torch

from . import _lib

KERNELS = {1: "router", 2: "gate_up", 3: "down"}
PHASES = ("start", "inputs in", "top-k done", "weights in", "end")


def clock_khz():
    """Ticks a millisecond of the stamps' clock on the current device."""
    k = ctypes.c_int(0)
    _lib.call("lmoe_timeline_clock_khz", ctypes.byref(k))
    return k.value


class Timeline:
    """``with Timeline(rows) as tl:`` arms the stamps into ``tl.buf`` [rows, 8] (int64, zeroed); on exit
    ``tl.launches`` lists (kernel name, first row, workgroups) of every stamped launch in launch order."""

    def __init__(self, rows, device="cuda"):
        self.buf = torch.zeros((rows, 8), dtype=torch.int64, device=device)
        self.launches = []

    def __enter__(self):
        _lib.call("lmoe_timeline_arm", _lib.ptr(self.buf), ctypes.c_longlong(self.buf.shape[0]))
        return self

    def __exit__(self, *exc):
        n = ctypes.c_int(0)
        _lib.call("lmoe_timeline_disarm", ctypes.byref(n))
        out = []
        for i in range(n.value):
            k, r0, nw = ctypes.c_int(0), ctypes.c_longlong(0), ctypes.c_int(0)
            _lib.call("lmoe_timeline_launch", i, ctypes.byref(k), ctypes.byref(r0), ctypes.byref(nw))
            out.append((KERNELS.get(k.value, str(k.value)), r0.value, nw.value))
        self.launches = out
        return False


def layer_phases(stamps, launches, khz):
    """One read of the stamp buffer (numpy [rows, 8]) over a stack's launches, three a layer (router, gate/up,
    down): for each layer and kernel, each phase's workgroup stamps in µs from the layer's first router workgroup
    start (phases a workgroup did not reach are dropped). Returns {kernel: {phase: [per-layer arrays]}}."""
    us = 1e3 / khz
    res = {name: {p: [] for p in PHASES} for name in KERNELS.values()}
    for l in range(0, len(launches) - 2, 3):
        names = [launches[l + i][0] for i in range(3)]
        if names != ["router", "gate_up", "down"]:
            raise ValueError(f"launches {l}..{l + 2} are {names}, not one layer's router, gate/up, down")
        r0, n0 = launches[l][1], launches[l][2]
        t0 = stamps[r0:r0 + n0, 0].min()
        for name, row0, nwg in launches[l:l + 3]:
            rows = stamps[row0:row0 + nwg]
            for i, p in enumerate(PHASES):
                v = rows[:, i]
                res[name][p].append((v[v != 0] - t0) * us)
    return res


def summary(res):
    """Per kernel and phase: the medians over layers of the first, median and last workgroup's stamp (µs from the
    layer's first router workgroup start)."""
    out = {}
    for name, ph in res.items():
        out[name] = {}
        for p, per_layer in ph.items():
            per_layer = [a for a in per_layer if a.size]
            if not per_layer:
                continue
            out[name][p] = {
                "first": round(float(np.median([a.min() for a in per_layer])), 2),
                "median": round(float(np.median([np.median(a) for a in per_layer])), 2),
                "last": round(float(np.median([a.max() for a in per_layer])), 2),
            }
    return out
