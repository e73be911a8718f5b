"""The routed-expert MoE layer on the CPU (numpy): router, grouping, expert chain, combine.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): the product path never imports this module.

Semantics follow the reference's MLX op sequence for a probability-routed block (stream_fast.py:4352-4377;
fused_router.py:568-583 ``glue_probs``; route_cuda.py:193-264 ``moe_probs`` / ``moe_tail``), with two deliberate
differences that the build's contract fixes:
  * ties in the top-k go to the LOWEST expert index (the reference's MLX argpartition puts the larger index
    first, route_cuda.py:14-16); selection is made on the fp32 logits, which orders experts exactly as the
    softmax probabilities do but without ties made by exp rounding;
  * everything is float32 (the reference rounds scores and the combine in bf16, route_cuda.py:245-263).
Grouping is the stable argsort of the flattened (token, k) expert ids (stream_fast.py:5466-5471,
gguf_experts.py:702-713). Expert outputs are the decode chain's (gguf_experts.py:444-447, 452-526):
h = silu(x . wg) * (x . wu), y = h . wd, all as an fp32 dequant-then-matmul.
"""
import numpy as np

from . import gguf


def softmax(logits):
    """float32 softmax over the last axis, max subtracted first (MLX's precise softmax order)."""
    z = np.asarray(logits, np.float32)
    m = z.max(axis=-1, keepdims=True)
    e = np.exp(z - m, dtype=np.float32)
    return (e / e.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)


def topk_ids(logits, k):
    """[..., E] logits -> [..., k] expert ids, best first; equal logits ordered by the lower expert index first."""
    z = np.asarray(logits, np.float32)
    if not 0 < k <= z.shape[-1]:
        raise ValueError(f"top-k {k} out of range for {z.shape[-1]} experts")
    return np.argsort(-z, axis=-1, kind="stable")[..., :k].astype(np.uint32)


def router(logits, k, norm):
    """The router of one MoE layer: (ids uint32 [..., k] best first, scores float32 [..., k]) with scores the
    softmax probabilities of the picked experts, renormalised to sum 1 when ``norm`` (route_cuda.py:280-288;
    stream_fast.py:4364-4370)."""
    ids = topk_ids(logits, k)
    g = softmax(logits)
    s = np.take_along_axis(g, ids.astype(np.int64), axis=-1).astype(np.float32)
    if norm:
        s = (s / s.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)
    return ids, s


def _tree(s):
    """Balanced binary tree sum over the last axis (a power of two long), neighbours first, in float32."""
    s = np.asarray(s, np.float32)
    while s.shape[-1] > 1:
        s = (s[..., 0::2] + s[..., 1::2]).astype(np.float32)
    return s[..., 0]


def _exact_products(x, w, H):
    x = np.asarray(x, np.float32).reshape(-1, H)
    w = np.asarray(w, np.float32).reshape(-1, H)
    return (w[None, :, :] * x[:, None, :]).astype(np.float32)  # [T, E, H]; f16 / bf16 products are exact in fp32


def router_logits_gemv(x, w):
    """Router logits [T, E] in the order of the per-layer router GEMV (larder_amd/csrc/router.hip k_router_gemv):
    thread i of 256 sums, in order, the products of its 8-element items i, i + 256, ... (item j covers elements
    [8 j, 8 j + 8)), starting from zero; each wavefront's 64 partials are added as a balanced binary tree in lane
    order; the four wavefronts' totals are added left to right. Exact for f16 / bf16 inputs, whose products fp32
    holds without rounding (each step then rounds once, as the GPU's fused multiply-add does); this is this build's
    order, not the reference's: its router is an MLX matmul (stream_fast.py:4352-4356) whose order MLX does not
    fix. Tokens go in chunks and the 256 threads' chains side by side, step by step, so a cfg5
    prefill (2048 tokens, 513 rows of 4096) runs in seconds."""
    x = np.asarray(x, np.float32)
    H = x.shape[-1]
    x = x.reshape(-1, H)
    w = np.asarray(w, np.float32).reshape(-1, H)
    T, E = x.shape[0], w.shape[0]
    nit = H // 8
    ni = -(-nit // 256)
    # element e of item it at [e, it], items padded to whole steps of 256 (the padding is never added: a thread
    # past the row's items keeps its chain as it is)
    pad = ni * 256
    xp = np.zeros((T, 8, pad), np.float32)
    xp[:, :, :nit] = x.reshape(T, nit, 8).transpose(0, 2, 1)
    wp = np.zeros((E, 8, pad), np.float32)
    wp[:, :, :nit] = w.reshape(E, nit, 8).transpose(0, 2, 1)
    out = np.empty((T, E), np.float32)
    chunk = max(1, (1 << 24) // (E * 256))
    prod = np.empty((min(chunk, T), E, 256), np.float32)
    for t0 in range(0, T, chunk):
        xc = xp[t0:t0 + chunk]
        n = xc.shape[0]
        acc = np.zeros((n, E, 256), np.float32)
        pr = prod[:n]
        for i in range(ni):
            m = min(256, nit - 256 * i)  # threads with an item at this step
            for e in range(8):
                np.multiply(xc[:, None, e, 256 * i:256 * i + m], wp[None, :, e, 256 * i:256 * i + m], out=pr[..., :m])
                np.add(acc[..., :m], pr[..., :m], out=acc[..., :m])
        waves = _tree(acc.reshape(n, E, 4, 64))
        out[t0:t0 + chunk] = (((waves[..., 0] + waves[..., 1]).astype(np.float32) + waves[..., 2]).astype(np.float32)
                              + waves[..., 3]).astype(np.float32)
    return out


def group_rows(ids, n_experts):
    """Flattened (token, k) rows bucketed by expert id: (counts [E], offsets [E + 1], order [R], inv [R]) with
    ``order`` the stable argsort of the flat ids (rows of one expert in flat order, experts ascending),
    ``inv[r]`` the position of flat row r in ``order``, and ids >= E (no such expert) placed after every valid
    row, in flat order, outside every expert's range (their outputs are zero, cpu_kern.cpp:316-318)."""
    flat = np.asarray(ids).reshape(-1).astype(np.int64)
    key = np.where((flat >= 0) & (flat < n_experts), flat, n_experts)
    order = np.argsort(key, kind="stable").astype(np.uint32)
    counts = np.bincount(key, minlength=n_experts + 1)[:n_experts].astype(np.uint32)
    offsets = np.zeros(n_experts + 1, np.uint32)
    offsets[1:] = np.cumsum(counts)
    inv = np.empty(len(flat), np.uint32)
    inv[order] = np.arange(len(flat), dtype=np.uint32)
    return counts, offsets, order, inv


def silu_mul(g, u):
    """SwiGLU: silu(g) * u = g * sigmoid(g) * u, float32 (gguf_experts.py:444-447)."""
    g = np.asarray(g, np.float32)
    with np.errstate(over="ignore"):
        sig = (np.float32(1.0) / (np.float32(1.0) + np.exp(-g, dtype=np.float32))).astype(np.float32)
    return (g * sig * np.asarray(u, np.float32)).astype(np.float32)


def sigmoid(v):
    v = np.asarray(v, np.float32)
    with np.errstate(over="ignore"):
        return (np.float32(1.0) / (np.float32(1.0) + np.exp(-v, dtype=np.float32))).astype(np.float32)


def dequant_experts(buf, t, which=None):
    """Experts of a [S, rows, row bytes] buffer as float32 [len(which), rows, cols] (all of them by default)."""
    buf = np.asarray(buf, np.uint8)
    if which is not None:
        buf = buf[np.asarray(which, np.int64)]
    return gguf.dequant_matrix(buf, t)


def gemv(x, w, slots, topk, types):
    """Every slot's expert output, unweighted, as gguf_experts.gemv defines it (gguf_experts.py:600-607):
    x [rows, H], slots [rows * topk] with slot s on x row s // topk, w = (gate, up, down) buffers
    [S, rows, row bytes] in ``types``; returns (h float32 [n, I], y float32 [n, H])."""
    x = np.asarray(x).astype(np.float32)
    slots = np.asarray(slots).reshape(-1).astype(np.int64)
    n = slots.size
    bg, bu, bd = w
    tg, tu, td = types
    inter = bg.shape[1]
    hid = x.shape[-1]
    h = np.zeros((n, inter), np.float32)
    y = np.zeros((n, hid), np.float32)
    ok = (slots >= 0) & (slots < bg.shape[0])
    for e in np.unique(slots[ok]):
        sel = np.nonzero(slots == e)[0]
        xr = x[sel // topk]
        wg = dequant_experts(bg, tg, [e])[0]
        wu = dequant_experts(bu, tu, [e])[0]
        wd = dequant_experts(bd, td, [e])[0]
        hh = silu_mul(xr @ wg.T, xr @ wu.T)
        h[sel] = hh
        y[sel] = hh @ wd.T
    return h, y


def combine(y, scores, shared=None, gate=None, residual=None):
    """out[t] = sum_j scores[t, j] * y[t, j] (+ sigmoid(gate[t]) * shared[t]) (+ residual[t]), float32
    (stream_fast.py:4372-4376; route_cuda.py:256-264)."""
    y = np.asarray(y, np.float32)
    s = np.asarray(scores, np.float32)
    out = np.einsum("tk,tkh->th", s, y, dtype=np.float32).astype(np.float32)
    if shared is not None:
        out = out + sigmoid(np.asarray(gate, np.float32).reshape(-1, 1)) * np.asarray(shared, np.float32)
    if residual is not None:
        out = out + np.asarray(residual, np.float32)
    return out.astype(np.float32)


def shared_expert(x, sg, su, sd, types):
    """The shared expert's output, h = silu(x . sg) * (x . su), y = h . sd; sg/su/sd [rows, row bytes]."""
    x = np.asarray(x, np.float32)
    wg = gguf.dequant_matrix(sg, types[0])
    wu = gguf.dequant_matrix(su, types[1])
    wd = gguf.dequant_matrix(sd, types[2])
    return silu_mul(x @ wg.T, x @ wu.T) @ wd.T


def layer(x, logits, w, types, k, norm, shared=None, shared_gate_w=None, residual=None):
    """One MoE layer as an fp32 dequant-then-matmul: router on ``logits`` [T, E], the top-k experts' SwiGLU
    chains, the weighted combine, plus (when ``shared`` = (sg, su, sd) buffers is given) the sigmoid-gated shared
    expert with gate logit x . shared_gate_w; returns (ids, scores, out float32 [T, H])."""
    x = np.asarray(x).astype(np.float32)
    ids, scores = router(logits, k, norm)
    _, y = gemv(x, w, ids.reshape(-1), k, types)
    T = x.shape[0]
    sh = gate = None
    if shared is not None:
        sh = shared_expert(x, *shared, types)
        gate = x @ np.asarray(shared_gate_w, np.float32).reshape(-1)
    out = combine(y.reshape(T, k, -1), scores, sh, gate, residual)
    return ids, scores, out


def rel_l2(got, want):
    """Relative L2 error ||got - want|| / ||want|| in float64."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    den = np.linalg.norm(want)
    return float(np.linalg.norm(got - want) / (den if den > 0 else 1.0))
