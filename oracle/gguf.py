"""ggml's Q4_0 / Q4_K block formats, and Q4_1 / Q5_K / Q6_K / Q8_0, on the CPU (numpy): dequant, validity check,
and deterministic quantizers.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): the product path never imports this module.

The dequant restates ggml's ``dequantize_row_*`` as the reference restates them in ``gguf_ref.py`` (Q4_0 / Q4_1:
gguf_ref.py:345-351; Q4_K / Q5_K: gguf_ref.py:253-276; Q6_K: :392-401; Q8_0: :354-355; the f16 field read:
:244-246), without fused multiply-adds. It is pinned by tests/test_oracle_golden.py against vectors that
tests/golden/make_golden.py (Q4_0, Q4_K) and tests/golden/make_golden_types.py (the other four) wrote from the
reference's own ``gguf_ref.ref_dequant``, and by closed-form special cases (d = 0, extreme nibbles, sign of d,
f16 subnormal d) in tests/test_oracle_props.py.

The quantizers are not in the reference (it only reads packs that llama.cpp wrote):
  * ``quantize_q4_0`` follows ggml's published ``quantize_row_q4_0_ref`` rule (d = signed-amax / -8,
    q = min(15, trunc(x / d + 8.5))), so it can be checked against ggml's reference behaviour;
  * ``quantize_q4_k`` is this build's own simple min/scale fit (not ggml's iterative ``make_qkx2_quants``); it
    only has to produce valid Q4_K blocks from Gaussian weights, and is checked by round trip; the Q4_1, Q5_K,
    Q6_K and Q8_0 quantizers are the same kind of plain fit, checked the same way.
"""
import numpy as np

# ggml type name -> (ggml type id, weights a block, bytes a block); the types this path implements
# (gguf_ref.py:8-15 lists all of them).
TYPES = {"Q4_0": (2, 32, 18), "Q4_K": (12, 256, 144), "Q4_1": (3, 32, 20), "Q5_K": (13, 256, 176),
         "Q6_K": (14, 256, 210), "Q8_0": (8, 32, 34)}
NAME_OF = {v[0]: k for k, v in TYPES.items()}


def row_bytes(t, n):
    """Bytes of one row of n weights in ggml type t (gguf_experts.py:35 gg_row)."""
    _, be, bb = TYPES[t]
    if n % be:
        raise ValueError(f"{t}: a row of {n} weights is not a whole number of {be}-weight blocks")
    return n // be * bb


def _f16(b, at):
    """The half at byte ``at`` of every block as float32 (gguf_ref.py:244-246)."""
    return np.ascontiguousarray(b[:, at:at + 2]).view(np.float16)[:, 0].astype(np.float32)


def _dq_q4_0(b):
    """Q4_0: byte j of qs holds weight j (low nibble) and j + 16 (high); w = (q - 8) * d (gguf_ref.py:345-351)."""
    qs = b[:, 2:18]
    q = np.concatenate([qs & 0xF, qs >> 4], axis=1).astype(np.int32)
    return (q - 8).astype(np.float32) * _f16(b, 0)[:, None]


def scale_min_k4(s):
    """ggml's get_scale_min_k4 for sub-blocks 0..7 of every block's 12 scale bytes -> (sc, m) float32 (n, 8)
    (gguf_ref.py:253-258)."""
    s = s.astype(np.uint8)
    sc = np.concatenate([s[:, 0:4] & 63, (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)], axis=1)
    m = np.concatenate([s[:, 4:8] & 63, (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)], axis=1)
    return sc.astype(np.float32), m.astype(np.float32)


def _dq_q4_k(b):
    """Q4_K: 256 weights; y = (d * sc_j) * q - (dmin * m_j) per 32-weight sub-block j, sub-block 2c in the low
    nibbles of qs[32c : 32c + 32] and 2c + 1 in the high ones (gguf_ref.py:261-276)."""
    n = b.shape[0]
    d, dmin = _f16(b, 0), _f16(b, 2)
    sc, m = scale_min_k4(b[:, 4:16])
    d1 = d[:, None] * sc
    m1 = dmin[:, None] * m
    ql = b[:, 16:144].reshape(n, 4, 32)
    q = np.stack([ql & 0xF, ql >> 4], axis=2).astype(np.float32)        # (n, 4, 2, 32): sub-block 2c + h
    y = d1.reshape(n, 4, 2, 1) * q - m1.reshape(n, 4, 2, 1)
    return y.reshape(n, 256)


def _dq_q4_1(b):
    """Q4_1: d at bytes 0-1, m at 2-3, qs at 4..19 (byte j: weight j low, j + 16 high); w = q * d + m
    (gguf_ref.py:345-351)."""
    qs = b[:, 4:20]
    q = np.concatenate([qs & 0xF, qs >> 4], axis=1).astype(np.float32)
    return q * _f16(b, 0)[:, None] + _f16(b, 2)[:, None]


def _dq_q8_0(b):
    """Q8_0: d at bytes 0-1, 32 int8 weights; w = q * d (gguf_ref.py:354-355)."""
    return np.ascontiguousarray(b[:, 2:34]).view(np.int8).astype(np.float32) * _f16(b, 0)[:, None]


def _dq_q5_k(b):
    """Q5_K: as Q4_K with the nibbles at bytes 48..175 and a fifth bit: bit j of qh[l] (bytes 16..47) adds 16 to
    weight l of sub-block j (gguf_ref.py:261-276)."""
    n = b.shape[0]
    d, dmin = _f16(b, 0), _f16(b, 2)
    sc, m = scale_min_k4(b[:, 4:16])
    d1 = d[:, None] * sc
    m1 = dmin[:, None] * m
    ql = b[:, 48:176].reshape(n, 4, 32)
    q = np.stack([ql & 0xF, ql >> 4], axis=2).astype(np.int32)          # (n, 4, 2, 32): sub-block 2c + h
    qh = b[:, 16:48].astype(np.int32)
    j = (2 * np.arange(4)[:, None] + np.arange(2)[None, :]).reshape(1, 4, 2, 1)
    q = q + 16 * ((qh[:, None, None, :] >> j) & 1)
    y = d1.reshape(n, 4, 2, 1) * q.astype(np.float32) - m1.reshape(n, 4, 2, 1)
    return y.reshape(n, 256)


def _dq_q6_k(b):
    """Q6_K: weight 128h + 32g + l (h < 2, g < 4, l < 32) = 6-bit q - 32 from nibble g // 2 of
    ql[64h + 32 (g % 2) + l] (bytes 0..127) and bits 2g, 2g + 1 of qh[32h + l] (bytes 128..191), times
    d * sc with sc the int8 at byte 192 + 8h + 2g + l // 16 and d the f16 at byte 208 (gguf_ref.py:392-401)."""
    n = b.shape[0]
    y = np.empty((n, 256), np.float32)
    d = _f16(b, 208)
    sc = np.ascontiguousarray(b[:, 192:208]).view(np.int8).astype(np.float32)
    l = np.arange(32)
    for h in range(2):
        for g in range(4):
            lo = (b[:, 64 * h + 32 * (g % 2) + l].astype(np.int32) >> (4 * (g // 2))) & 0xF
            hi = (b[:, 128 + 32 * h + l].astype(np.int32) >> (2 * g)) & 3
            q = ((lo | (hi << 4)) - 32).astype(np.float32)
            s = sc[:, 8 * h + 2 * g + l // 16]
            y[:, 128 * h + 32 * g + l] = (d[:, None] * s) * q
    return y


_DQ = {"Q4_0": _dq_q4_0, "Q4_K": _dq_q4_k, "Q4_1": _dq_q4_1, "Q8_0": _dq_q8_0, "Q5_K": _dq_q5_k,
       "Q6_K": _dq_q6_k}


def dequant(raw, t):
    """float32 weights of ``raw`` (bytes or a uint8 array of whole blocks) in ggml type t, flattened in row order."""
    _, be, bb = TYPES[t]
    b = np.frombuffer(raw, np.uint8) if isinstance(raw, (bytes, bytearray, memoryview)) else np.asarray(raw, np.uint8)
    if b.size % bb:
        raise ValueError(f"{t}: {b.size} bytes is not a whole number of {bb}-byte blocks")
    with np.errstate(over="ignore", invalid="ignore"):
        return _DQ[t](b.reshape(-1, bb)).reshape(-1).astype(np.float32, copy=False)


def dequant_matrix(buf, t):
    """[..., rows, row bytes] uint8 in type t -> [..., rows, row length] float32."""
    buf = np.asarray(buf, np.uint8)
    _, be, bb = TYPES[t]
    n = buf.shape[-1] // bb * be
    return dequant(buf.reshape(-1), t).reshape(buf.shape[:-1] + (n,))


# Byte offsets of each type's f16 fields (d, and dmin), as gguf_ref.HALVES (gguf_ref.py:557-562).
HALVES = {"Q4_0": (0,), "Q4_K": (0, 2), "Q4_1": (0, 2), "Q5_K": (0, 2), "Q6_K": (208,), "Q8_0": (0,)}


def valid(b, t):
    """ggml_validate_row_data's check for these types: every f16 scale finite (gguf_ref.py:564-581)."""
    b = np.asarray(b, np.uint8).reshape(-1, TYPES[t][2])
    h = np.concatenate([np.ascontiguousarray(b[:, a:a + 2]).view("<u2") for a in HALVES[t]], axis=1)
    return not ((h & 0x7C00) == 0x7C00).any()


def quantize_q4_0(w):
    """float weights [..., n] (n % 32 == 0) -> Q4_0 blocks [..., n / 32 * 18] uint8, ggml's quantize_row_q4_0_ref
    rule in float32: the first weight of largest magnitude sets d = max / -8, id = 1 / d (0 if d == 0),
    q = min(15, trunc(x * id + 8.5)), byte j = q[j] | q[j + 16] << 4, d stored as f16 (round to nearest even)."""
    w = np.asarray(w, np.float32)
    lead, n = w.shape[:-1], w.shape[-1]
    if n % 32:
        raise ValueError("Q4_0 rows must be a multiple of 32 weights")
    x = w.reshape(-1, 32)
    at = np.argmax(np.abs(x), axis=1)                       # first of the largest magnitude, as ggml's strict <
    mx = x[np.arange(len(x)), at]
    d = (mx / np.float32(-8.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, np.float32(1.0)), np.float32(0.0))
    inv = inv.astype(np.float32)
    v = (x * inv[:, None]).astype(np.float32) + np.float32(8.5)
    q = np.minimum(15, np.trunc(v).astype(np.int32)).astype(np.uint8)
    out = np.empty((len(x), 18), np.uint8)
    out[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:18] = q[:, :16] | (q[:, 16:] << 4)
    return out.reshape(lead + (n // 32 * 18,))


def quantize_q4_k(w):
    """float weights [..., n] (n % 256 == 0) -> Q4_K blocks [..., n / 256 * 144] uint8 by a plain min/scale fit:
    sub-block j gets scale (max - min) / 15 and min -min(x, 0); the super-block's d and dmin are the largest of
    those over 63 (stored f16); the 6-bit sc_j, m_j round against the stored f16 d, dmin and each weight takes
    q = clip(round((x + dmin m_j) / (d sc_j)), 0, 15). Scales pack as ggml's get_scale_min_k4 reads them."""
    w = np.asarray(w, np.float32)
    lead, n = w.shape[:-1], w.shape[-1]
    if n % 256:
        raise ValueError("Q4_K rows must be a multiple of 256 weights")
    x = w.reshape(-1, 8, 32)
    nb = x.shape[0]
    lo = np.minimum(x.min(axis=2), 0.0).astype(np.float32)
    hi = x.max(axis=2).astype(np.float32)
    scale = ((hi - lo) / np.float32(15.0)).astype(np.float32)
    mins = (-lo).astype(np.float32)
    d16 = (scale.max(axis=1) / np.float32(63.0)).astype(np.float16)
    m16 = (mins.max(axis=1) / np.float32(63.0)).astype(np.float16)
    d, dm = d16.astype(np.float32), m16.astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(d[:, None] > 0, np.rint(scale / d[:, None]), 0)
        m = np.where(dm[:, None] > 0, np.rint(mins / dm[:, None]), 0)
    sc = np.clip(sc, 0, 63).astype(np.uint8)
    m = np.clip(m, 0, 63).astype(np.uint8)
    dj = d[:, None] * sc.astype(np.float32)
    mj = dm[:, None] * m.astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(dj[:, :, None] > 0, np.rint((x + mj[:, :, None]) / dj[:, :, None]), 0)
    q = np.clip(q, 0, 15).astype(np.uint8)                     # (nb, 8, 32)
    out = np.zeros((nb, 144), np.uint8)
    out[:, 0:2] = d16.view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = m16.view(np.uint8).reshape(-1, 2)
    s = np.zeros((nb, 12), np.uint8)
    s[:, 0:4] = (sc[:, 0:4] & 63) | ((sc[:, 4:8] >> 4) << 6)
    s[:, 4:8] = (m[:, 0:4] & 63) | ((m[:, 4:8] >> 4) << 6)
    s[:, 8:12] = (sc[:, 4:8] & 0xF) | ((m[:, 4:8] & 0xF) << 4)
    out[:, 4:16] = s
    qs = q.reshape(nb, 4, 2, 32)
    out[:, 16:144] = (qs[:, :, 0, :] | (qs[:, :, 1, :] << 4)).reshape(nb, 128)
    return out.reshape(lead + (n // 256 * 144,))


def _rows(w, be, t):
    w = np.asarray(w, np.float32)
    if w.shape[-1] % be:
        raise ValueError(f"{t} rows must be a multiple of {be} weights")
    return w.shape[:-1], w.shape[-1], w.reshape(-1, be)


def _safe_div(a, b):
    with np.errstate(divide="ignore", invalid="ignore"):
        return np.where(b != 0, a / np.where(b != 0, b, 1), 0)


def quantize_q4_1(w):
    """Q4_1 by a min/max fit per 32 weights: m = min (f16), d = (max - m) / 15 (f16),
    q = clip(round((x - m) / d), 0, 15)."""
    lead, n, x = _rows(w, 32, "Q4_1")
    m16 = x.min(axis=1).astype(np.float16)
    d16 = ((x.max(axis=1) - m16.astype(np.float32)) / np.float32(15.0)).astype(np.float16)
    q = np.clip(np.rint(_safe_div(x - m16.astype(np.float32)[:, None], d16.astype(np.float32)[:, None])), 0, 15)
    q = q.astype(np.uint8)
    out = np.empty((len(x), 20), np.uint8)
    out[:, 0:2] = d16.view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = m16.view(np.uint8).reshape(-1, 2)
    out[:, 4:20] = q[:, :16] | (q[:, 16:] << 4)
    return out.reshape(lead + (n // 32 * 20,))


def quantize_q8_0(w):
    """Q8_0: d = max|x| / 127 (f16), q = clip(round(x / d), -127, 127)."""
    lead, n, x = _rows(w, 32, "Q8_0")
    d16 = (np.abs(x).max(axis=1) / np.float32(127.0)).astype(np.float16)
    q = np.clip(np.rint(_safe_div(x, d16.astype(np.float32)[:, None])), -127, 127).astype(np.int8)
    out = np.empty((len(x), 34), np.uint8)
    out[:, 0:2] = d16.view(np.uint8).reshape(-1, 2)
    out[:, 2:34] = q.view(np.uint8)
    return out.reshape(lead + (n // 32 * 34,))


def quantize_q5_k(w):
    """Q5_K by the Q4_K fit with 31 levels: qs nibbles as Q4_K's, the fifth bits in qh (bit j of byte l for
    weight l of sub-block j)."""
    lead, n, x = _rows(w, 256, "Q5_K")
    x = x.reshape(-1, 8, 32)
    nb = x.shape[0]
    lo = np.minimum(x.min(axis=2), 0.0).astype(np.float32)
    scale = ((x.max(axis=2) - lo) / np.float32(31.0)).astype(np.float32)
    mins = (-lo).astype(np.float32)
    d16 = (scale.max(axis=1) / np.float32(63.0)).astype(np.float16)
    m16 = (mins.max(axis=1) / np.float32(63.0)).astype(np.float16)
    d, dm = d16.astype(np.float32), m16.astype(np.float32)
    sc = np.clip(np.rint(_safe_div(scale, d[:, None])), 0, 63).astype(np.uint8)
    m = np.clip(np.rint(_safe_div(mins, dm[:, None])), 0, 63).astype(np.uint8)
    dj = d[:, None] * sc.astype(np.float32)
    mj = dm[:, None] * m.astype(np.float32)
    q = np.clip(np.rint(_safe_div(x + mj[:, :, None], dj[:, :, None])), 0, 31).astype(np.uint8)   # (nb, 8, 32)
    out = np.zeros((nb, 176), np.uint8)
    out[:, 0:2] = d16.view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = m16.view(np.uint8).reshape(-1, 2)
    out[:, 4:8] = (sc[:, 0:4] & 63) | ((sc[:, 4:8] >> 4) << 6)
    out[:, 8:12] = (m[:, 0:4] & 63) | ((m[:, 4:8] >> 4) << 6)
    out[:, 12:16] = (sc[:, 4:8] & 0xF) | ((m[:, 4:8] & 0xF) << 4)
    qh = np.zeros((nb, 32), np.uint8)
    for j in range(8):
        qh |= ((q[:, j, :] >> 4) & 1) << j
    out[:, 16:48] = qh
    ql = (q & 0xF).reshape(nb, 4, 2, 32)
    out[:, 48:176] = (ql[:, :, 0, :] | (ql[:, :, 1, :] << 4)).reshape(nb, 128)
    return out.reshape(lead + (n // 256 * 176,))


def quantize_q6_k(w):
    """Q6_K: per 16 weights s = max|x| / 31, d = max(s) / 127 (f16), sc = round(s / d) (int8),
    q = clip(round(x / (d sc)), -32, 31) + 32 split into ql nibbles and qh 2-bit fields as _dq_q6_k reads them."""
    lead, n, x = _rows(w, 256, "Q6_K")
    nb = x.shape[0]
    x16 = x.reshape(nb, 16, 16)
    s = (np.abs(x16).max(axis=2) / np.float32(31.0)).astype(np.float32)
    d16 = (s.max(axis=1) / np.float32(127.0)).astype(np.float16)
    d = d16.astype(np.float32)
    sc = np.clip(np.rint(_safe_div(s, d[:, None])), -128, 127).astype(np.int8)
    ds = d[:, None] * sc.astype(np.float32)
    q = np.clip(np.rint(_safe_div(x16, ds[:, :, None])), -32, 31).astype(np.int32) + 32      # (nb, 16, 16)
    q = q.reshape(nb, 256)
    out = np.zeros((nb, 210), np.uint8)
    l = np.arange(32)
    for h in range(2):
        for g in range(4):
            v = q[:, 128 * h + 32 * g + l]
            out[:, 64 * h + 32 * (g % 2) + l] |= ((v & 0xF) << (4 * (g // 2))).astype(np.uint8)
            out[:, 128 + 32 * h + l] |= ((v >> 4) << (2 * g)).astype(np.uint8)
    out[:, 192:208] = sc.view(np.uint8)
    out[:, 208:210] = d16.view(np.uint8).reshape(-1, 2)
    return out.reshape(lead + (n // 256 * 210,))


QUANTIZE = {"Q4_0": quantize_q4_0, "Q4_K": quantize_q4_k, "Q4_1": quantize_q4_1, "Q8_0": quantize_q8_0,
            "Q5_K": quantize_q5_k, "Q6_K": quantize_q6_k}


def random_experts(rng, n, rows, cols, t, std=0.02):
    """n experts [n, rows, row bytes] uint8 of type t quantized from Gaussian weights N(0, std^2) drawn as
    float32 from ``rng`` (numpy Generator) in [n, rows, cols] order."""
    w = (rng.standard_normal((n, rows, cols), dtype=np.float32) * np.float32(std)).astype(np.float32)
    return QUANTIZE[t](w)
