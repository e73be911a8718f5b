"""Router and combine of a probability-routed MoE block on MI355X: the call surface of the reference's
route_cuda.probs / route_cuda.tail (route_cuda.py:280-298) over torch tensors.

    probs(logits, k, norm) -> (inds, scores)
    tail(y, scores, shared, gate) -> out
    route(gates, mask, slot_of, lam, tau, k, lim=None, slots=True) -> (inds, ok, rhs)   (route_cuda.py:158-178)
    bias_probs(logits, slot_of, lam, tau, k, lim, norm) -> (inds, scores)               (route_cuda.py:306-417)

Differences from the reference kernels, by this build's contract: in probs() ties in the top-k go to the LOWEST
expert index (route_cuda.py:14-16 breaks them toward the larger one), any E up to 1024 and k up to 32 (not only
256 / 8), and scores are float32 (the reference rounds them to the logits' bf16). route() and bias_probs() keep the
reference's rule (larger index) and dtypes, because their callers compare against CacheBiasedMoE's MLX ops. ``inds`` keep the reference's layout: the
last k of an ascending ranking (best expert last, route_cuda.py:230-233).
"""
import torch

from ._lib import call, dcode, ptr, stream


def topk(logits, k, norm):
    """logits (..., E) -> (ids int32 (..., k) best first, scores float32 (..., k))."""
    lg = logits.contiguous()
    E = lg.shape[-1]
    T = lg.numel() // E
    ids = torch.empty(lg.shape[:-1] + (k,), dtype=torch.int32, device=lg.device)
    scores = torch.empty(lg.shape[:-1] + (k,), dtype=torch.float32, device=lg.device)
    call("lmoe_router_topk", ptr(lg), dcode(lg.dtype), T, E, k, int(bool(norm)), ptr(ids), ptr(scores), stream())
    return ids, scores


def probs(logits, k, norm):
    """softmax(logits) then the top k, as route_cuda.probs returns them (route_cuda.py:280-288): inds int32
    (..., k) in ascending rank (best last) and their float32 softmax probabilities, renormalised to sum 1 when
    ``norm``."""
    ids, scores = topk(logits, k, norm)
    return ids.flip(-1).contiguous(), scores.flip(-1).contiguous()


def tail(y, scores, shared, gate):
    """(y * scores[..., None]).sum(-2) + sigmoid(gate) * shared (route_cuda.py:291-298): y (..., T, k, D),
    scores (..., T, k), shared (..., T, D) float32 or None, gate (..., T, 1) or None; out in y's dtype."""
    t, k, d = y.shape[-3:]
    yy = y.reshape(t * k, d).contiguous()
    inv = torch.arange(t * k, dtype=torch.int32, device=y.device)
    sc = scores.reshape(t, k).to(torch.float32).contiguous()
    out = torch.empty(y.shape[:-2] + (d,), dtype=y.dtype, device=y.device)
    sh = gt = None
    if shared is not None:
        sh = shared.reshape(t, d).to(torch.float32).contiguous()
        gt = gate.reshape(t).to(torch.float32).contiguous()
    call("lmoe_combine_sorted", ptr(yy), dcode(yy.dtype), ptr(inv), ptr(sc), t, k, d, ptr(sh), ptr(gt), 1, None, 0,
         ptr(out), dcode(out.dtype), stream())
    return out


def _route_call(gates, mask, slot_of, lam, tau, k, lim, softmax, norm, want_slots, want_scores):
    g = gates.contiguous()
    E = g.shape[-1]
    T = g.numel() // E
    dev = g.device
    inds = torch.empty(g.shape[:-1] + (k,), dtype=torch.int32, device=dev)
    ok = torch.empty(1, dtype=torch.int32, device=dev) if want_slots else None
    rhs = torch.empty(g.shape[:-1] + (k,), dtype=torch.int32, device=dev) if want_slots else None
    scores = torch.empty(g.shape[:-1] + (k,), dtype=g.dtype, device=dev) if want_scores else None
    m = None if mask is None else mask.to(device=dev, dtype=torch.float32).contiguous()
    so = None if slot_of is None else slot_of.to(device=dev, dtype=torch.int32).contiguous()
    call("lmoe_route_bias", ptr(g), dcode(g.dtype), T, E, k, ptr(m), ptr(so), int(lim if lim is not None else 0),
         float(lam), float(tau), int(softmax), int(bool(norm)), ptr(inds), ptr(ok), ptr(rhs), ptr(scores),
         stream())
    return inds, ok, rhs, scores


def route(gates, mask, slot_of, lam, tau, k, lim=None, slots=True):
    """route_cuda.route (route_cuda.py:158-178): CacheBiasedMoE's cache-biased selection. gates (..., T, E) float32 /
    bfloat16 / float16; mask [E] float32, or None with ``lim`` (table mode: the mask is 0 <= slot_of < lim);
    slot_of [E] int32 -> (inds int32 (..., T, k) ascending, best last, ok int32 [1], rhs int32 (..., T, k) =
    max(slot_of[inds], 0)); slots=False -> (inds,). Ties go to the larger index and the bias and budget
    arithmetic follow the reference's (MLX's) dtypes and order; see include/larder_moe.h lmoe_route_bias."""
    if mask is None and lim is None:
        raise ValueError("route needs a mask or, in table mode, lim")
    inds, ok, rhs, _ = _route_call(gates, mask, slot_of, lam, tau, k, lim, False, False, slots, False)
    return (inds, ok, rhs) if slots else (inds,)


def bias_probs(logits, slot_of, lam, tau, k, lim, norm):
    """route_cuda.bias_probs (route_cuda.py:306-417): softmax of logits (..., T, E), then the table-mode cache-biased
    route and budget, then the picked gates (renormalised in output order when ``norm``) -> (inds int32 (..., T, k),
    scores (..., T, k) in the logits' dtype). Any E <= 1024 and k <= 32 (the reference: 256 and 8)."""
    inds, _, _, scores = _route_call(logits, None, slot_of, lam, tau, k, lim, True, norm, False, True)
    return inds, scores
