"""Known-answer check of liblarder_moe.so on the device: run once a process and device, before the first call that
launches work there (the reference checks its kernels when they are first used, gguf_experts.py:661-680; here the
inputs are fixed and the answers recorded). Inputs are built from integer formulas; the answers are the oracle's:
  * lmoe_dequant of Q4_0 and Q4_K experts must give the recorded bits (SHA-256 of the float32 output);
  * the decode chain (lmoe_gemv_gate_up + lmoe_gemv_down_combine) on a Q4_0 and a Q4_K expert, and the grouped MFMA
    path on the Q4_K one, must give the recorded outputs within 2e-3 relative L2 (sampled entries and the norm).
A failure raises RuntimeError naming the check: no result of a library that fails it is trusted. LMOE_SELF_CHECK=0
skips the check."""
import hashlib

import numpy as np
import torch

# (rows, cols) of each projection: Q4_0 at H = I = 64, Q4_K at H = I = 256
SHAPES = {"Q4_0": 64, "Q4_K": 256}
# every STRIDE-th entry of y is recorded, with the norm of all of it
STRIDE = {"Q4_0": 4, "Q4_K": 16}
BAR = 2e-3

# SHA-256 (first 16 hex digits) of the float32 dequant of the gate expert, and (sampled y, |y|) of the chain
EXPECT_DEQUANT = {"Q4_0": "2c375755c65b64d3", "Q4_K": "96fd9b15569e563f"}
EXPECT_Y = {
    "Q4_0": ([-0.00642979145, -0.045458544, 0.0346243121, 0.0186462402, -0.0460736081, -0.0838032588, 0.0365185291,
              0.00699354615, 0.054474514, -0.0309777111, -0.00241997186, 0.0459403992, -0.00316444784, -0.0389312059,
              -0.000367608853, 0.0175356828], 0.344096036),
    "Q4_K": ([0.139530048, 0.000587314367, 1.44997954, 1.34656954, 0.417522699, 0.449097008, 0.190221012, 0.529129267,
              0.740898132, 0.177317977, 0.283749372, 0.270931542, 0.395813107, 0.51586616, 0.157478213, 0.980767548],
             10.0083933),
}


def _bytes(n, salt):
    i = np.arange(n, dtype=np.uint64) + np.uint64(salt)
    return ((i * np.uint64(2654435761) >> np.uint64(13)) & np.uint64(0xFF)).astype(np.uint8)


def blocks(t, rows, cols, salt):
    """One expert [1, rows, row bytes] of type t: pseudo-random quant bytes with small exact f16 scales."""
    if t == "Q4_0":
        nb = rows * cols // 32
        b = _bytes(nb * 18, salt).reshape(nb, 18)
        d = (2.0 ** -6 * (1 + (np.arange(nb) % 7) / 8)).astype(np.float16)
        b[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        return b.reshape(1, rows, cols // 32 * 18)
    nb = rows * cols // 256
    b = _bytes(nb * 144, salt).reshape(nb, 144)
    d = (2.0 ** -12 * (1 + (np.arange(nb) % 5) / 4)).astype(np.float16)
    dmin = (2.0 ** -13 * (1 + (np.arange(nb) % 3) / 4)).astype(np.float16)
    b[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    b[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    return b.reshape(1, rows, cols // 256 * 144)


def inputs(t):
    """(x [1, H] float32, exact in f16; gate, up, down experts) of the check for block type t."""
    n = SHAPES[t]
    x = (((np.arange(n) * 37) % 19 - 9) / 8.0).astype(np.float32).reshape(1, n)
    w = tuple(blocks(t, n, n, salt) for salt in (11, 23, 37))
    return x, w


def digest(a):
    return hashlib.sha256(np.ascontiguousarray(a, np.float32).tobytes()).hexdigest()[:16]


def summary(t, y):
    """(sampled entries, norm) of a chain output row y [H]."""
    y = np.asarray(y, np.float64).reshape(-1)
    return [float(v) for v in y[::STRIDE[t]]], float(np.linalg.norm(y))


def verify(t, dq_digest, y_rows):
    """Raise RuntimeError unless the dequant digest and every output row in y_rows match the recorded answers."""
    if dq_digest != EXPECT_DEQUANT[t]:
        raise RuntimeError(f"larder_amd self-check: {t} dequant gave {dq_digest}, not the recorded "
                           f"{EXPECT_DEQUANT[t]}")
    want, norm = EXPECT_Y[t]
    want = np.asarray(want, np.float64)
    for label, y in y_rows:
        got, gnorm = summary(t, y)
        err = float(np.linalg.norm(np.asarray(got) - want) / max(np.linalg.norm(want), 1e-30))
        if not (err < BAR and abs(gnorm - norm) <= BAR * norm):
            raise RuntimeError(f"larder_amd self-check: {t} {label} is off the recorded answer (sampled rel L2 "
                               f"{err:.2e}, norm {gnorm:.6g} against {norm:.6g})")


def run(device=None):
    """The check on the current device (raises RuntimeError on a mismatch)."""
    from . import grouped
    from ._lib import call, dcode, ptr, qcode, stream
    dev = torch.device("cuda", torch.cuda.current_device() if device is None else device)
    for t in ("Q4_0", "Q4_K"):
        x, w = inputs(t)
        n = SHAPES[t]
        wd = tuple(torch.from_numpy(b).to(dev) for b in w)
        s = torch.zeros(1, dtype=torch.int32, device=dev)
        q = torch.empty((1, n, n), dtype=torch.float32, device=dev)
        call("lmoe_dequant", ptr(wd[0]), qcode(t), 1, n, n, ptr(s), 1, ptr(q), dcode(torch.float32), stream())
        xd = torch.from_numpy(x).to(dev).half()
        h = torch.empty((1, n), dtype=torch.float32, device=dev)
        y = torch.empty((1, n), dtype=torch.float32, device=dev)
        call("lmoe_gemv_gate_up", ptr(xd), dcode(xd.dtype), ptr(s), 1, 1, ptr(wd[0]), ptr(wd[1]), qcode(t),
             qcode(t), 1, n, n, ptr(h), stream())
        call("lmoe_gemv_down_combine", ptr(h), ptr(s), None, 1, 1, ptr(wd[2]), qcode(t), 1, n, n, None, None, 0,
             None, 0, ptr(y), dcode(torch.float32), stream())
        rows = [("decode chain", y[0])]
        if t == "Q4_K":  # the grouped GEMMs take H and I in multiples of 256 / 128
            yy = grouped.expert_rows(xd.repeat(2, 1).contiguous(), wd, torch.zeros(2, dtype=torch.int32, device=dev),
                                     (t,) * 3, torch.float32)
            rows += [("grouped path", yy[0]), ("grouped path", yy[1])]
        torch.cuda.synchronize(dev)
        verify(t, digest(q.cpu().numpy()), [(label, r.cpu().numpy()) for label, r in rows])
