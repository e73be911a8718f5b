"""Prefill routing pinned bit-exact from x and the router weight.

The reference routes every chunk with one op sequence (stream_fast.py:4352-4370: the gate matmul, softmax, top-k).
Here the prefill router is an MFMA GEMM whose summation order nothing restates; lmoe_router_gemm_refine keeps its
speed and makes the picks exact: the candidates its proven error bound leaves are recomputed in the decode router's
fixed order (k_router_gemv), which the oracle restates (oracle.moe.router_logits_gemv, pinned by
test_oracle_router_order.py). So the ids here are checked against the oracle's top-k of ITS OWN logits from x and
Wr, for every token, never against the GPU's logits.
"""
import numpy as np
import pytest
import torch

from oracle import moe

pytestmark = pytest.mark.gpu

BAR = 2e-3


def host(t):
    return t.detach().cpu().numpy()


def _layer(cfg, seed):
    from larder_amd import workloads
    g = torch.Generator(device="cuda").manual_seed(seed)
    return workloads.make_layer(cfg, g), g


def _check_routing(L, x, B, cfg):
    """ids (all tokens) against the oracle's top-k of the fixed-order logits from x and Wr, and the shared gate's
    logit and slots, bit for bit; the scores and the candidate counts."""
    xs = host(x.float())  # f16 / bf16 values, exact in float32
    wr = host(L.wr.float())
    want_lg = moe.router_logits_gemv(xs, wr)
    k, E = cfg["k"], cfg["E"]
    want_ids = moe.topk_ids(want_lg, k)
    got_ids = host(B.ids_ext)[:, :k].astype(np.uint32)
    bad = np.nonzero((got_ids != want_ids).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} of {len(got_ids)} tokens' ids differ, first {bad[:5].tolist()}"
    # the logits row: the fixed-order logit where the pick recomputed it (every candidate whose bound interval meets
    # another's), the GEMM's elsewhere, within the GEMM's error of the fixed order everywhere
    got_lg = host(B.logits)
    assert np.allclose(got_lg, want_lg, rtol=1e-4, atol=1e-4 * np.abs(want_lg).max())
    if L.shared is not None:
        want_gate = moe.router_logits_gemv(xs, host(L.wsg.float()).reshape(1, -1))[:, 0]
        assert np.array_equal(host(B.gate).view(np.uint32), want_gate.view(np.uint32))
        if B.fold:
            m = L.n_shared
            assert (host(B.ids_ext)[:, k:] == E + np.arange(m)).all()
            assert np.allclose(host(B.scores_ext)[:, k:], 1 / (1 + np.exp(-want_gate[:, None].astype(np.float64))),
                               rtol=1e-6)
    # scores: the softmax terms of the picks (exact fixed-order logits), renormalised when norm
    _, want_sc = moe.router(want_lg, k, cfg["norm"])
    assert np.allclose(host(B.scores_ext)[:, :k], want_sc, rtol=2e-5, atol=1e-7)
    nc = host(B.n_cand)
    assert (nc >= k).all()
    return want_lg, nc


CASES = {
    # BASELINE cfg5 prefill: E 512, top-10, the shared expert folded in, bf16 activations, 2048 tokens
    "cfg5_T2048": (dict(H=4096, E=512, k=10, I=512, norm=True, Is=512, types=("Q4_K",) * 3), 2048, torch.bfloat16),
    # cfg1: E 60, top-4 without renorm, the 5632-wide shared expert folded in as four slices
    "cfg1_T150": (dict(H=2048, E=60, k=4, I=1408, norm=False, Is=5632, types=("Q4_0",) * 3), 150, torch.float16),
    # cfg2's layer with its router weight, 1024 tokens
    "cfg2_T1024": (dict(H=2048, E=128, k=8, I=768, norm=True, Is=0, types=("Q4_0",) * 3), 1024, torch.bfloat16),
    # a single token
    "cfg2_T1": (dict(H=2048, E=128, k=8, I=768, norm=True, Is=0, types=("Q4_0",) * 3), 1, torch.float16),
}


@pytest.mark.parametrize("name", list(CASES))
def test_prefill_routing_bit_exact_from_x(name):
    from larder_amd import grouped
    cfg, T, xdt = CASES[name]
    L, g = _layer(cfg, 31)
    x = torch.randn((T, cfg["H"]), generator=g, device="cuda").to(xdt)
    B = grouped.PrefillBuffers(L, T)
    out = torch.empty((T, cfg["H"]), dtype=torch.float32, device="cuda")
    grouped.prefill(L, x, B, out)
    torch.cuda.synchronize()
    _, nc = _check_routing(L, x, B, cfg)
    print(f"{name}: candidates a token mean {nc.mean():.2f} max {nc.max()} (k {cfg['k']})", flush=True)
    assert nc.mean() <= cfg["k"] + 8  # the bound is tight enough to leave a few extra candidates, not all experts


def test_prefill_routing_unfolded_shared_gate():
    """A shared expert that runs apart (not folded): the gate logit the combine uses is the fixed-order one."""
    from larder_amd import grouped
    from larder_amd.layer import MoELayer
    cfg = dict(H=2048, E=60, k=4, I=1408, norm=False, Is=5632, types=("Q4_0",) * 3)
    L, g = _layer(cfg, 32)
    U = MoELayer(L.wg, L.wu, L.wd, L.types, L.k, L.norm, wr=L.wr, shared=L.shared, wsg=L.wsg, fold_shared=False)
    T = 64
    x = torch.randn((T, cfg["H"]), generator=g, device="cuda").half()
    B = grouped.PrefillBuffers(U, T)
    assert not B.fold
    out = torch.empty((T, cfg["H"]), dtype=torch.float32, device="cuda")
    grouped.prefill(U, x, B, out)
    torch.cuda.synchronize()
    _check_routing(U, x, B, cfg)


@pytest.mark.parametrize("kind", ["duplicate_rows", "one_ulp_rows", "tiny_x", "zero_rows"])
def test_prefill_routing_planted_near_ties(kind):
    """Router rows built so that logits tie exactly (duplicated rows: the lower index must win), differ by one f16 unit
    of one weight (a gap far inside the GEMM's error bound: the fixed order must decide), or tokens whose logits are
    all tiny or all zero: the picks still equal the oracle's."""
    from larder_amd import grouped
    cfg = dict(H=2048, E=128, k=8, I=512, norm=True, Is=0, types=("Q4_0",) * 3)
    L, g = _layer(cfg, 33)
    wr = L.wr.clone()
    T = 256
    x = torch.randn((T, cfg["H"]), generator=g, device="cuda").half()
    if kind == "duplicate_rows":
        for dst, src in ((7, 3), (9, 3), (100, 50), (127, 0)):
            wr[dst] = wr[src]
    elif kind == "one_ulp_rows":
        bits = wr.view(torch.int16)
        for dst, src, col in ((7, 3, 5), (9, 3, 1000), (100, 50, 2047), (127, 0, 0)):
            bits[dst] = bits[src]
            bits[dst, col] += 1
        # and make those rows the likely winners: scale them up
        wr[[3, 7, 9, 0, 127, 50, 100]] *= 4
    elif kind == "tiny_x":
        x = (x.float() * 1e-6).half()  # f16 subnormals among them
    elif kind == "zero_rows":
        wr[10:20] = 0
        x[:8] = 0  # all logits zero: ids 0..7 by the tie rule
    L.wr = wr.contiguous()
    L._router_k = L._router_norms = None
    B = grouped.PrefillBuffers(L, T)
    out = torch.empty((T, cfg["H"]), dtype=torch.float32, device="cuda")
    grouped.prefill(L, x, B, out)
    torch.cuda.synchronize()
    _check_routing(L, x, B, cfg)
    if kind == "zero_rows":
        assert (host(B.ids_ext)[:8] == np.arange(8)).all()


def test_router_gemm_within_the_bound():
    """The bound's premise, measured: the MFMA router GEMM's logits against the exact dot of the f16 operands, in
    units of the bound's term g * sum |x_i w_i| (g = (H / ks + ks + 64) 2^-23 for ks K slices of the GEMM; here
    ks = 8, 7x tighter than a bound over all H terms in one order); the worst token x expert must stay far below 1.
    Rows with heavy cancellation (x and w of alternating signs) are included."""
    from larder_amd import _lib, grouped
    cfg = dict(H=4096, E=128, k=8, I=512, norm=True, Is=0, types=("Q4_K",) * 3)
    L, g = _layer(cfg, 34)
    T = 512
    x = torch.randn((T, cfg["H"]), generator=g, device="cuda").half()
    alt = torch.where(torch.arange(cfg["H"], device="cuda") % 2 == 0, 1.0, -1.0)
    x[:16] = (alt * 3.0).half()
    wr = L.wr.clone()
    wr[:16] = (alt * 0.5 + torch.randn((16, cfg["H"]), generator=g, device="cuda") * 1e-3).half()
    L.wr = wr
    L._router_k = L._router_norms = None
    B = grouped.PrefillBuffers(L, T)
    xh = torch.empty((T, cfg["H"]), dtype=torch.float16, device="cuda")
    _lib.call("lmoe_to_gemm_f16", _lib.ptr(x), _lib.F16, x.numel(), _lib.ptr(xh), _lib.stream())
    lg = torch.empty((T, cfg["E"]), dtype=torch.float32, device="cuda")
    _lib.call("lmoe_router_gemm", _lib.ptr(xh), T, cfg["H"], _lib.ptr(L.router_gemm_weight()), cfg["E"], 0,
              _lib.ptr(B.rws), _lib.ptr(lg), None, _lib.stream())
    torch.cuda.synchronize()
    xd = host(x).astype(np.float64)
    wd = host(L.wr).astype(np.float64)
    exact = xd @ wd.T
    absdot = np.abs(xd) @ np.abs(wd).T
    ks = _lib.lib().lmoe_router_gemm_ksplit(T, cfg["H"], cfg["E"])
    assert ks == 8
    gfac = (cfg["H"] // ks + ks + 64) * 2.0 ** -23
    ratio = np.abs(host(lg).astype(np.float64) - exact) / (gfac * absdot)
    print(f"router GEMM error / bound term: max {ratio.max():.3g}, mean {ratio.mean():.3g}", flush=True)
    assert ratio.max() < 0.25
    # and the picks of this layer, through the refine, against the oracle
    out = torch.empty((T, cfg["H"]), dtype=torch.float32, device="cuda")
    grouped.prefill(L, x, B, out)
    torch.cuda.synchronize()
    _check_routing(L, x, B, cfg)
