"""CPU oracle (test infrastructure only) for the cache-biased router: the reference's route_cuda.route and
route_cuda.bias_probs (route_cuda.py:42-121, 158-178, 306-417), which reproduce CacheBiasedMoE._select's MLX ops
(tests/test_route_cuda.py:28-41) in one kernel.

Per row of gates g [E] (dtype T: float32, float16 or bfloat16; every value below is a float32 holding a T value):
  spread = T(max(g) - min(g)); ls = T(T(lam) * spread)
  rank = float(g) + float(ls) * m            fp32, multiply then add, m = mask[e] (table mode: 0 <= slot_of < lim)
  inds = the k largest of rank, MLX's stable ascending sort read from the back: ties go to the LARGER index, and
         the k come in ascending order (best last)                          (route_cuda.py:14-16, 79-96) 
  budget (tau > 0 and lam > 0): honest = the same on g; m_h, m_b = the k gates summed in T in MLX's
         row_reduce_simple order (route_cuda.py:17-19, 98-113); back = T(m_h - m_b) > T(T(tau) * m_h)
  inds = honest if back; slots = slot_of[inds]; ok = all(slots >= 0); rhs = max(slots, 0)
bias_probs: gates = T(softmax(logits)) first, table mode, then scores = the picked gates, and with norm each
divided by their sum taken in pick order from 0 in T (route_cuda.py:386-393).

The softmax is exact (float64, then rounded to T). The reference's kernel uses CUDA's __expf, whose results this
oracle does not reproduce: gates can differ from it by one T ulp, so bias_probs parity is to that tolerance.
"""
import numpy as np

__all__ = ["round_to", "route", "bias_probs", "topk_mlx", "row_reduce_sum", "softmax_gates"]


def round_to(x, dt):
    """float32 values rounded to dt ('f32', 'f16', 'bf16'; round to nearest even), returned as float32."""
    x = np.asarray(x, dtype=np.float32)
    if dt == "f32":
        return x.copy()
    if dt == "f16":
        return x.astype(np.float16).astype(np.float32)
    if dt == "bf16":
        u = x.view(np.uint32).astype(np.uint64)
        nan = np.isnan(x)
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
        out = (r & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
        return np.where(nan, x, out).astype(np.float32)
    raise ValueError(dt)


def topk_mlx(rank, k):
    """The last k of a stable ascending sort by (value, index): ties to the larger index, ascending order."""
    rank = np.asarray(rank, dtype=np.float32)
    idx = np.arange(rank.shape[0])
    order = np.lexsort((idx, rank.astype(np.float64)))  # by value, then by index, both ascending
    return order[-k:].astype(np.int64)


def row_reduce_sum(vals, dt):
    """Sum of the k values (float32 holding dt values) as the reference's budget does (route_cuda.py:36-37, 98-113):
    32 lanes, lane l adds elements l*N .. l*N+N-1 in order from 0 (N = 16 / sizeof(T)), each add rounded to dt,
    then lanes combine by xor 16, 8, 4, 2, 1 (all lanes end equal; lane 0's is the sum)."""
    vals = np.asarray(vals, dtype=np.float32)
    k = vals.shape[0]
    n = 4 if dt == "f32" else 8
    acc = np.zeros(32, dtype=np.float32)
    for lane in range(32):
        a = np.float32(0.0)
        for i in range(n):
            j = lane * n + i
            v = vals[j] if j < k else np.float32(0.0)
            a = round_to(np.float32(a + v), dt)[()]
        acc[lane] = a
    for m in (16, 8, 4, 2, 1):
        nxt = acc.copy()
        for lane in range(32):
            nxt[lane] = round_to(np.float32(acc[lane] + acc[lane ^ m]), dt)[()]
        acc = nxt
    return np.float32(acc[0])


def _select_row(g, m, lam, tau, k, dt):
    g = np.asarray(g, dtype=np.float32)
    spread = round_to(np.float32(g.max() - g.min()), dt)[()]
    ls = round_to(np.float32(round_to(np.float32(lam), dt)[()] * spread), dt)[()]
    rank = (g + (np.float32(ls) * m.astype(np.float32)).astype(np.float32)).astype(np.float32)
    inds = topk_mlx(rank, k)
    if tau > 0.0 and lam > 0.0:
        honest = topk_mlx(g, k)
        mh = row_reduce_sum(g[honest], dt)
        mb = row_reduce_sum(g[inds], dt)
        d = round_to(np.float32(mh - mb), dt)[()]
        r = round_to(np.float32(round_to(np.float32(tau), dt)[()] * mh), dt)[()]
        if d > r:
            inds = honest
    return inds


def route(gates, dt, mask, slot_of, lam, tau, k, lim=None):
    """gates [T, E] float32 holding dt values; mask [E] float32, or None with lim (table mode: the mask is
    0 <= slot_of < lim); slot_of [E] int32 -> (inds [T, k] uint32, ok bool, rhs [T, k] int32)."""
    gates = np.asarray(gates, dtype=np.float32)
    slot_of = np.asarray(slot_of, dtype=np.int64)
    if mask is None:
        m = ((slot_of >= 0) & (slot_of < lim)).astype(np.float32)
    else:
        m = np.asarray(mask, dtype=np.float32)
    inds = np.stack([_select_row(g, m, lam, tau, k, dt) for g in gates])
    slots = slot_of[inds]
    return inds.astype(np.uint32), bool((slots >= 0).all()), np.maximum(slots, 0).astype(np.int32)


def softmax_gates(logits, dt):
    """softmax over the last axis, exact in float64, rounded to dt."""
    x = np.asarray(logits, dtype=np.float64)
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return round_to((e / e.sum(axis=-1, keepdims=True)).astype(np.float32), dt)


def bias_probs(logits, dt, slot_of, lam, tau, k, lim, norm):
    """logits [T, E] float32 holding dt values -> (inds [T, k] uint32, scores [T, k] float32 holding dt values):
    softmax, the table-mode route, the picked gates, renormalised in pick order when norm."""
    g = softmax_gates(logits, dt)
    inds, _, _ = route(g, dt, None, slot_of, lam, tau, k, lim)
    scores = np.take_along_axis(g, inds.astype(np.int64), axis=-1).astype(np.float32)
    if norm:
        out = np.empty_like(scores)
        for r in range(scores.shape[0]):
            s = np.float32(0.0)
            for j in range(k):
                s = round_to(np.float32(s + scores[r, j]), dt)[()]
            out[r] = round_to((scores[r] / s).astype(np.float32), dt)
        scores = out
    return inds, scores
