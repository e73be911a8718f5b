"""CPU oracle (test infrastructure only) for the trunk's 4-bit affine matmul of T bf16 rows, the reference's
route_cuda.qmv_rows (route_cuda.py:460-541), which reproduces MLX 0.32.4's one-row qmv kernel for every row.

Weights are MLX's affine 4-bit layout: w uint32 [N, K / 8] with element j of a word at bits 4j, scales and biases
bf16 [N, K / G]; weight = q * s + b. Per output row n and input row t (route_cuda.py:464-511):
  * 32 lanes; lane l takes elements idx = base + 16 l .. idx + 15 for base = 0, 512, ... (idx < K);
  * the 16 weights in bf16: m = bf16(q * s), w = bf16(m + b) (one group: G % 16 == 0);
  * 16 bf16 accumulators a lane, slot e holding elements idx + e over the bases: a_e = bf16(x * w + a_e), one
    rounding (a bf16 fused multiply-add);
  * s = the 16 slots summed in float32 in slot order from 0, then the xor butterfly over the 32 lanes (16, 8, 4,
    2, 1) in float32; out = bf16(s).
Every value below is a float32 array holding bf16 values. bf16(q s) and bf16(m + b) are exact in float64 before
their one rounding (8-bit operands); the fused multiply-add rounds once through fma_bf16.
"""
import numpy as np

__all__ = ["bf16", "fma_bf16", "qmv_rows", "quantize_affine4", "dequant_affine4", "unpack4"]


def bf16(x):
    """Values (any float array) rounded once to bf16, round to nearest even, returned as float32: with x = m 2^e
    (0.5 <= |m| < 1), bf16 keeps 8 significant bits, so the result is rint(x / 2^(e - 8)) 2^(e - 8) (numpy's rint
    rounds half to even; the exponent is held at -125 and above, bf16's subnormal range)."""
    x = np.asarray(x, dtype=np.float64)
    _, e = np.frexp(x)
    ulp = np.ldexp(1.0, np.maximum(e, -125) - 8)
    return (np.rint(x / ulp) * ulp).astype(np.float32)


def fma_bf16(x, w, a):
    """bf16(x w + a) with one rounding, for bf16 values x, w, a: the product is exact in float64 (16 significant
    bits); the sum s = p + a is float64-rounded with its error e recovered exactly (TwoSum), and e breaks the tie
    when s falls exactly on a bf16 rounding midpoint (the one case a second rounding could get wrong)."""
    p = np.asarray(x, np.float64) * np.asarray(w, np.float64)
    a = np.asarray(a, np.float64)
    s = p + a
    bb = s - p
    e = (p - (s - bb)) + (a - bb)
    _, ex = np.frexp(s)
    ulp = np.ldexp(1.0, np.maximum(ex, -125) - 8)
    lo = np.floor(s / ulp) * ulp
    tie = (s - lo) == ulp / 2
    r = bf16(s).astype(np.float64)
    r = np.where(tie & (e > 0), lo + ulp, r)
    r = np.where(tie & (e < 0), lo, r)
    return r.astype(np.float32)


def unpack4(w, K):
    """uint32 [N, K / 8] -> int [N, K] of 4-bit values, element j of a word at bits 4j."""
    w = np.asarray(w, dtype=np.uint32)
    sh = (4 * np.arange(8, dtype=np.uint32))[None, None, :]
    return ((w[:, :, None] >> sh) & 15).reshape(w.shape[0], K).astype(np.int64)


def qmv_rows(x, w, scales, biases, G):
    """x [T, K] (bf16 values), w uint32 [N, K / 8], scales / biases [N, K / G] (bf16 values) -> out [T, N] (bf16
    values), the reference kernel's arithmetic step for step."""
    x = np.asarray(x, dtype=np.float32)
    T, K = x.shape
    N = w.shape[0]
    q = unpack4(w, K).astype(np.float64)                                  # [N, K]
    s = np.repeat(np.asarray(scales, np.float64), G, axis=1)[:, :K]
    b = np.repeat(np.asarray(biases, np.float64), G, axis=1)[:, :K]
    wd = bf16(bf16(q * s).astype(np.float64) + b).astype(np.float64)     # [N, K]
    out = np.empty((T, N), np.float32)
    for t in range(T):
        acc = np.zeros((N, 32, 16), np.float32)                           # slot accumulators, bf16 values
        for base in range(0, K, 512):
            idx = base + 16 * np.arange(32)
            live = idx < K
            for e in range(16):
                col = np.minimum(idx + e, K - 1)
                new = fma_bf16(x[t, col][None, :], wd[:, col], acc[:, :, e])
                acc[:, :, e] = np.where(live[None, :], new, acc[:, :, e])
        ssum = np.zeros((N, 32), np.float32)
        for e in range(16):
            ssum = (ssum + acc[:, :, e]).astype(np.float32)
        for m in (16, 8, 4, 2, 1):
            ssum = (ssum + ssum[:, np.arange(32) ^ m]).astype(np.float32)
        out[t] = bf16(ssum[:, 0])
    return out


def dequant_affine4(w, scales, biases, G):
    """The weights q * s + b in float64 (no rounding), [N, K]."""
    K = w.shape[1] * 8
    q = unpack4(w, K).astype(np.float64)
    s = np.repeat(np.asarray(scales, np.float64), G, axis=1)
    b = np.repeat(np.asarray(biases, np.float64), G, axis=1)
    return q * s + b


def quantize_affine4(w, G):
    """float weights [N, K] -> (w uint32 [N, K / 8], scales, biases bf16 values [N, K / G]) by a min/max fit a
    group: b = bf16(min), s = bf16((max - min) / 15), q = clip(round((x - b) / s), 0, 15)."""
    w = np.asarray(w, np.float32)
    N, K = w.shape
    g = w.reshape(N, K // G, G)
    lo = bf16(g.min(axis=2))
    s = bf16((g.max(axis=2) - lo) / 15.0)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(s[..., None] > 0, np.rint((g - lo[..., None]) / s[..., None]), 0)
    q = np.clip(q, 0, 15).astype(np.uint32).reshape(N, K // 8, 8)
    packed = np.zeros((N, K // 8), np.uint32)
    for j in range(8):
        packed |= q[:, :, j] << np.uint32(4 * j)
    return packed, s.astype(np.float32), lo.astype(np.float32)
