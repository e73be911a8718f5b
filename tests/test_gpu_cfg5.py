"""Configuration 5: H 4096, 512 routed experts, top-10 renormalised, I 512, a shared
expert (Is 512) with a sigmoid gate, all in GGUF Q4_K, at T = 1 (decode chain) and T = 2048 (grouped path); plus the
device Q4_K quantizer that builds these packs, bit-exact against the CPU oracle's.

Layer outputs are checked against the oracle's fp32 dequant-then-matmul on the experts the tokens touch (each
token's output depends only on its own experts, so a token sample is exact); ids bit-exact."""
import numpy as np
import pytest
import torch

from oracle import gguf, moe

pytestmark = pytest.mark.gpu

BAR = 2e-3


def host(t):
    return t.detach().cpu().numpy()


def test_quantize_q4_k_bit_exact():
    from larder_amd import _lib
    rng = np.random.default_rng(21)
    w = rng.standard_normal((96, 512)).astype(np.float32) * 0.02
    w[0] = 0.0                                    # zero super-block: d = dmin = 0
    w[1, :256] = 0.37                             # constant positive
    w[2, :256] = -0.11                            # constant negative
    w[3, 256:] = np.linspace(-1, 1, 256)          # one wide super-block
    w[4, :32] = 1e-30                             # a sub-block of tiny values
    w[5] *= 1000.0                                # large magnitudes
    for dt in (torch.float32, torch.float16, torch.bfloat16):
        wt = torch.from_numpy(w).cuda().to(dt)
        out = torch.empty((96, 512 // 256 * 144), dtype=torch.uint8, device="cuda")
        _lib.call("lmoe_quantize_q4_k", _lib.ptr(wt), _lib.dcode(dt), 96, 512, _lib.ptr(out), _lib.stream())
        want = gguf.quantize_q4_k(host(wt.float()))
        got = host(out)
        assert (got == want).all(), (dt, np.argwhere(got != want)[:5])
        assert gguf.valid(got.reshape(-1, 144), "Q4_K")


def _layer(seed):
    from larder_amd import workloads
    g = torch.Generator(device="cuda").manual_seed(seed)
    return workloads.make_layer(workloads.CONFIGS[5], g), g


def _oracle_subset(L, xs, logits, cfg):
    """moe.layer restricted to the experts the tokens touch (same result: other experts contribute nothing)."""
    ids, _ = moe.router(logits, cfg["k"], cfg["norm"])
    used = np.unique(ids)
    sel = torch.from_numpy(used.astype(np.int64)).cuda()
    w = tuple(host(b.index_select(0, sel)) for b in (L.wg, L.wu, L.wd))
    remap = np.zeros(cfg["E"], np.int64)
    remap[used] = np.arange(len(used))
    # gemv over the compact expert set, then the same combine as moe.layer
    _, y = moe.gemv(xs, w, remap[ids].reshape(-1), cfg["k"], cfg["types"])
    _, scores = moe.router(logits, cfg["k"], cfg["norm"])
    sh = moe.shared_expert(xs, *(host(b[0]) for b in L.shared), cfg["types"])
    gate = xs @ host(L.wsg.float())
    out = moe.combine(y.reshape(len(xs), cfg["k"], -1), scores, sh, gate)
    return ids, out


def test_cfg5_decode_T1():
    from larder_amd import layer as lay, workloads
    cfg = workloads.CONFIGS[5]
    L, g = _layer(5)
    x = torch.randn((1, cfg["H"]), generator=g, device="cuda").half()
    B = lay.DecodeBuffers(L, 1)
    out = torch.empty((1, cfg["H"]), dtype=torch.float32, device="cuda")
    lay.decode(L, x, B, out)
    torch.cuda.synchronize()
    xs = host(x.float())
    # routing pinned from x: the router GEMV's fixed order restated, bit for bit, then the oracle's own top-k
    want_lg = moe.router_logits_gemv(host(x), host(L.wr))
    lg = host(B.logits)
    assert np.array_equal(lg[:, :cfg["E"]].view(np.uint32), want_lg.view(np.uint32))
    want_gate = moe.router_logits_gemv(host(x), host(L.wsg).reshape(1, -1))
    assert np.array_equal(lg[:, cfg["E"]:].view(np.uint32), want_gate.view(np.uint32))
    ids, want = _oracle_subset(L, xs, want_lg, cfg)
    assert (host(B.ids).astype(np.uint32) == ids).all()
    assert moe.rel_l2(host(out), want) < BAR


def test_cfg5_prefill_T2048_sampled():
    from larder_amd import grouped, workloads
    cfg = workloads.CONFIGS[5]
    L, g = _layer(6)
    T = 2048
    x = torch.randn((T, cfg["H"]), generator=g, device="cuda").bfloat16()
    B = grouped.PrefillBuffers(L, T)
    out = torch.empty((T, cfg["H"]), dtype=torch.float32, device="cuda")
    grouped.prefill(L, x, B, out)
    torch.cuda.synchronize()
    # routing pinned from x and Wr: the oracle's fixed-order logits (the decode router's order, which the prefill's
    # exact pick reproduces), their top-k against every token's ids
    xs_all = host(x.float())
    lg = moe.router_logits_gemv(xs_all, host(L.wr.float()))
    ids_all, _ = moe.router(lg, cfg["k"], cfg["norm"])
    assert (host(B.ids).astype(np.uint32) == ids_all).all()
    rng = np.random.default_rng(1)
    sample = np.sort(rng.choice(T, 24, replace=False))
    xs = xs_all[sample]
    _, want = _oracle_subset(L, xs, lg[sample], cfg)
    got = host(out)[sample]
    assert moe.rel_l2(got, want) < BAR
    num = np.linalg.norm(got - want, axis=1)
    assert (num / np.linalg.norm(want, axis=1)).max() < 1e-2


@pytest.mark.parametrize("T", [1, 3])
def test_cfg5_decode_folded_shared_matches_unfolded(T):
    """The shared expert folded into the decode kernels as slot k (3 launches a layer) against the same layer with
    it run apart (5 launches): ids equal, the slot's id E and score sigmoid(gate logit), outputs within the bar;
    and the folded layer against the oracle (test_cfg5_decode_T1 above runs the folded form as well)."""
    from larder_amd import layer as lay, workloads
    cfg = workloads.CONFIGS[5]
    L, g = _layer(8)
    assert L.folded is not None
    U = lay.MoELayer(L.wg, L.wu, L.wd, L.types, L.k, L.norm, wr=L.wr, shared=L.shared, wsg=L.wsg,
                     fold_shared=False)
    assert U.folded is None
    x = torch.randn((T, cfg["H"]), generator=g, device="cuda").half()
    res = torch.randn((T, cfg["H"]), generator=g, device="cuda").half()
    outs = []
    for layer in (L, U):
        B = lay.DecodeBuffers(layer, T)
        out = torch.empty((T, cfg["H"]), dtype=torch.float32, device="cuda")
        lay.decode(layer, x, B, out, residual=res)
        torch.cuda.synchronize()
        outs.append((host(out), host(B.ids).copy(), B))
    (of, idf, Bf), (ou, idu, _) = outs
    assert (idf == idu).all()
    lg = host(Bf.logits)
    assert (host(Bf.ids_ext)[:, -1] == cfg["E"]).all()
    assert np.allclose(host(Bf.scores_ext)[:, -1], 1 / (1 + np.exp(-lg[:, cfg["E"]])), rtol=1e-5)
    r = host(res.float())
    assert moe.rel_l2(of - r, ou - r) < BAR
    xs = host(x.float())
    ids, want = _oracle_subset(L, xs, lg[:, :cfg["E"]], cfg)
    assert moe.rel_l2(of - r, want) < BAR
