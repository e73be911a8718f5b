"""Router and combine of a probability-routed MoE block on MI355X: the call surface of the reference's
route_cuda.probs / route_cuda.tail (route_cuda.py:280-298) over torch tensors.

    probs(logits, k, norm) -> (inds, scores)
    tail(y, scores, shared, gate) -> out

Differences from the reference kernels, by this build's contract: ties in the top-k go to the LOWEST expert index
(route_cuda.py:14-16 breaks them toward the larger one), any E up to 1024 and k up to 32 (not only 256 / 8), and
scores are float32 (the reference rounds them to the logits' bf16). ``inds`` keep the reference's layout: the
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
