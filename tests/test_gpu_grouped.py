"""GPU parity of the grouped (prefill / batched decode) path against the CPU oracle, through the C ABI.

Bars: expert ids and groupings bit-exact, ties to the lowest expert index; outputs
within 2e-3 relative L2 of an fp32 dequant-then-matmul (oracle.moe). Every row is also held to a per-row bar, so
one wrong row or tile cannot hide inside a large tensor."""
import numpy as np
import pytest
import torch

from oracle import gguf, moe

pytestmark = pytest.mark.gpu

BAR = 2e-3
ROW_BAR = 1e-2

_W = {}


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.detach().cpu().numpy()


def experts(types, H, I, E, seed):
    """CPU-quantized experts (gate, up, down), cached across parametrized cases."""
    key = (types, H, I, E, seed)
    if key not in _W:
        rng = np.random.default_rng(seed)
        _W[key] = tuple(gguf.random_experts(rng, E, r, c, t) for (r, c), t in zip(((I, H), (I, H), (H, I)), types))
    return _W[key]


def ragged_slots(rng, R, E):
    """One expert takes ~40% of the rows (several m-tiles), one ~10%, experts 1 and 2 none, the rest scattered."""
    s = rng.integers(3, E, R)
    s[: int(R * 0.4)] = 0
    s[int(R * 0.4): int(R * 0.5)] = E - 1
    return s[rng.permutation(R)].astype(np.int32)


def rows_ok(got, want, bar=ROW_BAR):
    num = np.linalg.norm(got.astype(np.float64) - want, axis=-1)
    den = np.maximum(np.linalg.norm(want.astype(np.float64), axis=-1), 1e-30)
    return float((num / den).max())


MIXES = [(("Q4_0",) * 3, 2048, 768, 8), (("Q4_K",) * 3, 1024, 512, 6), (("Q4_0",) * 3, 512, 1408, 5),
         (("Q4_K",) * 3, 4096, 256, 4), (("Q4_0",) * 3, 256, 128, 4)]


@pytest.mark.parametrize("types,H,I,E", MIXES)
@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16, torch.float32])
def test_expert_rows_vs_oracle(types, H, I, E, xdt):
    """gguf_experts.dense's contract: each row through its own slot, unweighted, rows in the caller's order."""
    from larder_amd import grouped
    w = experts(types, H, I, E, H + I)
    rng = np.random.default_rng(H * 3 + I)
    R = 333
    slots = ragged_slots(rng, R, E)
    slots[5] = E + 2                                     # no such expert: a zero row
    x = dev(rng.standard_normal((R, H)).astype(np.float32)).to(xdt)
    y = grouped.expert_rows(x, tuple(dev(b) for b in w), dev(slots), types, torch.float32)
    xs = host(x.float().half().float())                  # the kernels meet x as f16
    _, want = moe.gemv(xs, w, slots, 1, types)
    got = host(y)
    assert (got[5] == 0).all()
    assert moe.rel_l2(got, want) < BAR
    keep = np.arange(R) != 5
    assert rows_ok(got[keep], want[keep]) < ROW_BAR


@pytest.mark.parametrize("types,tile,ks", [(("Q4_0",) * 3, "32", "2"), (("Q4_0",) * 3, "64", ""),
                                           (("Q4_K",) * 3, "128", ""), (("Q4_K",) * 3, "32", "")])
def test_knobs_force_tiling(types, tile, ks, monkeypatch):
    """LMOE_TILE_ROWS / LMOE_KSPLIT force the grouped path's tiling (here against the rule's choice for 40 rows over
    6 experts), and the result stays within the bar."""
    from larder_amd import grouped
    H, I, E = (2048, 768, 6) if types[0] == "Q4_0" else (1024, 512, 6)
    w = experts(types, H, I, E, 77)
    rng = np.random.default_rng(78)
    R = 40
    slots = rng.integers(0, E, R).astype(np.int32)
    monkeypatch.setenv("LMOE_TILE_ROWS", tile)
    monkeypatch.setenv("LMOE_KSPLIT", ks)
    assert grouped.pick_tile_rows(R, E, types) == int(tile)
    if ks:
        assert grouped.pick_ksplit(R, E, int(tile), H) == int(ks)
    x = dev(rng.standard_normal((R, H)).astype(np.float32)).half()
    y = grouped.expert_rows(x, tuple(dev(b) for b in w), dev(slots), types, torch.float32)
    _, want = moe.gemv(host(x.float()), w, slots, 1, types)
    assert moe.rel_l2(host(y), want) < BAR
    assert rows_ok(host(y), want) < ROW_BAR


def test_large_outputs_f16_limit_and_f32_y():
    """Expert outputs past f16's range (down scales multiplied by a power of two): the default f16 y turns them into
    inf, the documented limit; PrefillBuffers(y_dtype=float32) and expert_rows with a bf16 / f32 out keep them
    finite and within the bar."""
    from larder_amd import grouped
    from larder_amd.layer import MoELayer
    types, H, I, E, T, k = ("Q4_0",) * 3, 2048, 768, 8, 32, 2
    rng = np.random.default_rng(90)
    wg, wu, wd = (gguf.random_experts(rng, E, r, c, "Q4_0") for r, c in ((I, H), (I, H), (H, I)))
    x = rng.standard_normal((T, H)).astype(np.float16)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    _, _, base = moe.layer(x.astype(np.float32), lg, (wg, wu, wd), types, k, True)
    f = 2.0 ** int(np.ceil(np.log2(2e5 / np.abs(base).max())))
    d = wd.reshape(-1, 18)[:, :2].copy().view(np.float16)
    assert np.isfinite(d.astype(np.float32) * f).all() and (np.abs(d.astype(np.float32) * f) < 65504).all()
    wd.reshape(-1, 18)[:, :2] = (d.astype(np.float32) * f).astype(np.float16).view(np.uint8)
    _, _, want = moe.layer(x.astype(np.float32), lg, (wg, wu, wd), types, k, True)
    assert np.abs(want).max() > 65504
    L = MoELayer(dev(wg), dev(wu), dev(wd), types, k, True)
    for y_dtype in (torch.float16, torch.float32):
        B = grouped.PrefillBuffers(L, T, y_dtype=y_dtype)
        out = torch.empty((T, H), dtype=torch.float32, device="cuda")
        grouped.prefill(L, dev(x), B, out, logits=dev(lg))
        got = host(out)
        if y_dtype == torch.float16:
            assert not np.isfinite(got).all()              # the f16 y's limit
        else:
            assert np.isfinite(got).all() and moe.rel_l2(got, want) < BAR
    slots = rng.integers(0, E, 40).astype(np.int32)
    xr = dev(rng.standard_normal((40, H)).astype(np.float16))
    _, yw = moe.gemv(host(xr.float()), (wg, wu, wd), slots, 1, types)
    assert np.abs(yw).max() > 65504
    for odt in (torch.float32, torch.bfloat16):
        y = host(grouped.expert_rows(xr, (dev(wg), dev(wu), dev(wd)), dev(slots), types, odt).float())
        ref = yw if odt == torch.float32 else host(torch.from_numpy(yw).bfloat16().float())   # out rounding
        assert np.isfinite(y).all() and moe.rel_l2(y, ref) < BAR


@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float32, torch.float16])
def test_to_gemm_f16_k_order(xdt):
    """lmoe_to_gemm_f16: every element rounded to f16 once and placed at its K-order position."""
    from larder_amd import grouped
    x = torch.randn((7, 160), device="cuda").to(xdt)
    got = grouped.as_gemm_f16(x)
    torch.cuda.synchronize()
    assert torch.equal(got[:, grouped.kperm_index(160)], x.half())


@pytest.mark.parametrize("cfgid,T,fold", [(5, 2048, True), (5, 300, True), (2, 8192, False), (2, 64, False),
                                         (1, 5, False)])
def test_router_gemm_topk_equals_the_two_steps(cfgid, T, fold):
    """lmoe_router_gemm_topk against lmoe_router_gemm + lmoe_router_topk(_shared): logits, gate logit, ids and scores
    bit for bit (split-K and not), and the ids are the oracle's top-k of those logits."""
    from larder_amd import _lib, grouped, workloads
    cfg = dict(workloads.CONFIGS[cfgid])
    if not fold:
        cfg["Is"] = 0
    g = torch.Generator(device="cuda").manual_seed(T + cfgid)
    L = workloads.make_layer(cfg, g)
    x = torch.randn((T, cfg["H"]), generator=g, device="cuda").bfloat16()
    xh = grouped.as_gemm_f16(x)
    E, k, ng = cfg["E"], cfg["k"], 1 if fold else 0
    m = L.n_shared if fold else 0
    ks = k + m
    f32, i32 = dict(dtype=torch.float32, device="cuda"), dict(dtype=torch.int32, device="cuda")
    nws = _lib.lib().lmoe_router_gemm_workspace_bytes(T, cfg["H"], E + ng)
    ws = torch.empty(max(nws // 4, 1), **f32)
    out = [[torch.empty((T, E), **f32), torch.empty(T, **f32), torch.empty((T, ks), **i32), torch.empty((T, ks), **f32)]
           for _ in range(2)]
    w = L.router_gemm_weight()
    st = _lib.stream()
    lg, gt, ids, sc = out[0]
    _lib.call("lmoe_router_gemm", _lib.ptr(xh), T, cfg["H"], _lib.ptr(w), E, ng, _lib.ptr(ws), _lib.ptr(lg),
              _lib.ptr(gt) if ng else None, st)
    if fold:
        _lib.call("lmoe_router_topk_shared", _lib.ptr(lg), T, E, k, int(cfg["norm"]), _lib.ptr(gt), m, _lib.ptr(ids),
                  _lib.ptr(sc), st)
    else:
        _lib.call("lmoe_router_topk", _lib.ptr(lg), _lib.F32, T, E, k, int(cfg["norm"]), _lib.ptr(ids), _lib.ptr(sc),
                  st)
    lg2, gt2, ids2, sc2 = out[1]
    _lib.call("lmoe_router_gemm_topk", _lib.ptr(xh), T, cfg["H"], _lib.ptr(w), E, ng, _lib.ptr(ws), _lib.ptr(lg2),
              _lib.ptr(gt2) if ng else None, k, int(cfg["norm"]), m, _lib.ptr(ids2), _lib.ptr(sc2), st)
    torch.cuda.synchronize()
    bits = lambda t: t.view(torch.int32)  # noqa: E731
    assert torch.equal(bits(lg), bits(lg2)) and torch.equal(ids, ids2) and torch.equal(bits(sc), bits(sc2))
    if ng:
        assert torch.equal(bits(gt), bits(gt2))
    assert np.array_equal(host(ids2)[:, :k].astype(np.uint32), moe.topk_ids(host(lg2), k))


@pytest.mark.parametrize("T,E,k,xdt", [(1, 60, 4, torch.bfloat16), (37, 128, 8, torch.float16),
                                        (513, 512, 10, torch.float32), (2048, 128, 8, torch.bfloat16)])
def test_topk_and_gemm_f16_equals_the_two_launches(T, E, k, xdt):
    """lmoe_topk_and_gemm_f16 against lmoe_router_topk + lmoe_to_gemm_f16: ids, scores and xh bit for bit (with tied
    rows), and the ids are the oracle's."""
    from larder_amd import _lib
    g = torch.Generator(device="cuda").manual_seed(T + E)
    lg = torch.randn((T, E), generator=g, device="cuda")
    lg[::3, : E // 2] = lg[::3, :1]                      # ties on every third row
    H = 2048
    x = torch.randn((T, H), generator=g, device="cuda").to(xdt)
    i32, f32 = dict(dtype=torch.int32, device="cuda"), dict(dtype=torch.float32, device="cuda")
    ids_a, sc_a, ids_b, sc_b = torch.empty((T, k), **i32), torch.empty((T, k), **f32), torch.empty((T, k), **i32), \
        torch.empty((T, k), **f32)
    xa, xb = (torch.empty((T, H), dtype=torch.float16, device="cuda") for _ in range(2))
    st = _lib.stream()
    _lib.call("lmoe_router_topk", _lib.ptr(lg), _lib.F32, T, E, k, 1, _lib.ptr(ids_a), _lib.ptr(sc_a), st)
    _lib.call("lmoe_to_gemm_f16", _lib.ptr(x), _lib.dcode(xdt), x.numel(), _lib.ptr(xa), st)
    _lib.call("lmoe_topk_and_gemm_f16", _lib.ptr(lg), _lib.F32, T, E, k, 1, _lib.ptr(ids_b), _lib.ptr(sc_b),
              _lib.ptr(x), _lib.dcode(xdt), x.numel(), _lib.ptr(xb), st)
    torch.cuda.synchronize()
    assert torch.equal(ids_a, ids_b) and torch.equal(sc_a.view(torch.int32), sc_b.view(torch.int32))
    assert torch.equal(xa.view(torch.int16), xb.view(torch.int16))
    assert np.array_equal(host(ids_b).astype(np.uint32), moe.topk_ids(host(lg), k))


@pytest.mark.parametrize("types,H,I,E", MIXES[:2])
def test_gate_up_h_matches_oracle(types, H, I, E):
    """h in grouped order against the oracle's h, element by element (f16 output rounding plus f16 weights)."""
    from larder_amd import grouped
    w = experts(types, H, I, E, H + I)
    rng = np.random.default_rng(5)
    T, k = 70, 3
    ids = rng.integers(0, E, (T, k)).astype(np.int32)
    ids[:20] = 0
    x = dev(rng.standard_normal((T, H)).astype(np.float16))
    G = grouped.Grouping(T * k, E).run(dev(ids.reshape(-1)))
    h = torch.empty((T * k, I), dtype=torch.float16, device="cuda")
    grouped.gate_up(x, G, k, dev(w[0]), dev(w[1]), types, h)
    order = host(G.order)
    hw, _ = moe.gemv(host(x.float()), w, ids.reshape(-1), k, types)
    got = host(grouped.from_kperm(h).float())
    assert moe.rel_l2(got, hw[order]) < BAR
    assert rows_ok(got, hw[order]) < ROW_BAR


def _device_layer(cfg, seed):
    from larder_amd import workloads
    g = torch.Generator(device="cuda").manual_seed(seed)
    return workloads.make_layer(cfg, g), g


@pytest.mark.parametrize("cfgid,T,xdt", [(2, 300, torch.bfloat16), (4, 64, torch.float16), (2, 1, torch.float16),
                                         (2, 129, torch.float32)])
def test_prefill_layer_vs_oracle(cfgid, T, xdt):
    """A whole layer from given logits (cfg3's skewed draw, cfg4's Zipf prior) with the residual fused."""
    from larder_amd import grouped, workloads
    cfg = workloads.CONFIGS[cfgid]
    L, g = _device_layer(cfg, 7 + T)
    lg = (workloads.zipf_logits if cfgid == 4 else workloads.skewed_logits)(T, cfg["E"], g)
    x = torch.randn((T, cfg["H"]), generator=g, device="cuda").to(xdt)
    B = grouped.PrefillBuffers(L, T)
    out = torch.empty((T, cfg["H"]), dtype=torch.float32, device="cuda")
    grouped.prefill(L, x, B, out, residual=x, logits=lg)
    torch.cuda.synchronize()
    xs = host(x.float().half().float())
    ids, scores, want = moe.layer(xs, host(lg), tuple(host(b) for b in (L.wg, L.wu, L.wd)), cfg["types"], cfg["k"],
                                  cfg["norm"], residual=host(x.float()))
    assert (host(B.ids).astype(np.uint32) == ids).all()
    assert np.allclose(host(B.scores), scores, rtol=2e-6, atol=1e-7)
    xr = host(x.float())
    assert moe.rel_l2(host(out) - xr, want - xr) < BAR
    assert rows_ok(host(out) - xr, want - xr) < ROW_BAR


def test_prefill_layer_cfg1_shared_expert():
    """Config 1's layer (E 60, top-4 without renorm, I 1408, shared 5632 + sigmoid gate) with router logits from
    the router weight."""
    from larder_amd import grouped, workloads
    cfg = workloads.CONFIGS[1]
    L, g = _device_layer(cfg, 3)
    T = 150
    x = torch.randn((T, cfg["H"]), generator=g, device="cuda").half()
    B = grouped.PrefillBuffers(L, T)
    out = torch.empty((T, cfg["H"]), dtype=torch.float32, device="cuda")
    grouped.prefill(L, x, B, out)
    torch.cuda.synchronize()
    xs = host(x.float())
    # routing pinned from x and Wr: the oracle's fixed-order logits (the decode router's order, which the prefill's
    # exact pick reproduces), not the GPU's
    lg = moe.router_logits_gemv(xs, host(L.wr.float()))
    assert moe.rel_l2(host(B.logits), xs @ host(L.wr.float()).T) < 1e-5
    ids, _, want = moe.layer(xs, lg, tuple(host(b) for b in (L.wg, L.wu, L.wd)), cfg["types"],
                             cfg["k"], cfg["norm"], shared=tuple(host(b[0]) for b in L.shared),
                             shared_gate_w=host(L.wsg.float()))
    assert (host(B.ids).astype(np.uint32) == ids).all()
    assert moe.rel_l2(host(out), want) < BAR
    assert rows_ok(host(out), want) < ROW_BAR


@pytest.mark.parametrize("cfgid,T", [(1, 150), (5, 96)])
def test_prefill_folded_shared_matches_apart(cfgid, T):
    """A shared expert folded into the grouped GEMMs (cfg1: four slices of the routed width, cfg5: one; slots
    k .. k + m - 1 of every token from lmoe_router_topk_shared) against the same layer with the shared expert run
    apart on a side stream: equal routed ids, the slots' ids E + j and sigmoid weights, outputs within the bar."""
    from larder_amd import grouped, workloads
    from larder_amd.layer import MoELayer
    cfg = dict(workloads.CONFIGS[cfgid])
    if cfgid == 5:
        cfg.update(E=64)
    L, g = _device_layer(cfg, 21)
    assert L.folded is not None and L.n_shared == cfg["Is"] // cfg["I"]
    U = MoELayer(L.wg, L.wu, L.wd, L.types, L.k, L.norm, wr=L.wr, shared=L.shared, wsg=L.wsg, fold_shared=False)
    x = torch.randn((T, cfg["H"]), generator=g, device="cuda").half()
    outs = []
    for layer in (L, U):
        B = grouped.PrefillBuffers(layer, T)
        assert B.fold == (layer is L)
        out = torch.empty((T, cfg["H"]), dtype=torch.float32, device="cuda")
        grouped.prefill(layer, x, B, out)
        torch.cuda.synchronize()
        outs.append((host(out), host(B.ids).copy(), B))
    (of, idf, Bf), (ou, idu, _) = outs
    assert (idf == idu).all()
    m = L.n_shared
    assert (host(Bf.ids_ext)[:, cfg["k"]:] == cfg["E"] + np.arange(m)).all()
    gate = host(Bf.gate)
    assert np.allclose(host(Bf.scores_ext)[:, cfg["k"]:], 1 / (1 + np.exp(-gate[:, None])), rtol=1e-5)
    assert moe.rel_l2(of, ou) < BAR
    lg = moe.router_logits_gemv(host(x.float()), host(L.wr.float()))  # routing pinned from x
    assert (host(Bf.ids).astype(np.uint32) == moe.topk_ids(lg, cfg["k"])).all()
    _, _, want = moe.layer(host(x.float()), lg, tuple(host(b) for b in (L.wg, L.wu, L.wd)), cfg["types"], cfg["k"],
                           cfg["norm"], shared=tuple(host(b[0]) for b in L.shared), shared_gate_w=host(L.wsg.float()))
    assert moe.rel_l2(of, want) < BAR
    assert rows_ok(of, want) < ROW_BAR


def test_prefill_matches_decode_chain():
    """The grouped path and the decode chain (separately checked against the oracle) agree on the same tokens."""
    from larder_amd import grouped, layer as lay, workloads
    cfg = workloads.CONFIGS[2]
    L, g = _device_layer(cfg, 11)
    T = 16
    x = torch.randn((T, cfg["H"]), generator=g, device="cuda").half()
    lg = workloads.skewed_logits(T, cfg["E"], g)
    out_g = torch.empty((T, cfg["H"]), dtype=torch.float32, device="cuda")
    out_d = torch.empty_like(out_g)
    B = grouped.PrefillBuffers(L, T)
    grouped.prefill(L, x, B, out_g, logits=lg)
    D = lay.DecodeBuffers(L, T)
    lay.decode(L, x, D, out_d, logits=lg)
    torch.cuda.synchronize()
    assert torch.equal(B.ids, D.ids)
    assert moe.rel_l2(host(out_g), host(out_d)) < BAR


def test_prefill_cfg3_full_size():
    """Config 3 at its full size (8192 bf16 tokens, top-8 of 128, skewed logits): ids and grouping bit-exact for all
    65,536 rows, and 48 sampled tokens against the oracle (tokens are independent, so the sample is exact)."""
    from larder_amd import grouped, workloads
    cfg = workloads.CONFIGS[3]
    L, g = _device_layer(cfg, 0)
    T, E, k = cfg["T"], cfg["E"], cfg["k"]
    lg = workloads.skewed_logits(T, E, g)
    x = torch.randn((T, cfg["H"]), generator=g, device="cuda").bfloat16()
    B = grouped.PrefillBuffers(L, T)
    out = torch.empty((T, cfg["H"]), dtype=torch.bfloat16, device="cuda")
    grouped.prefill(L, x, B, out, logits=lg)
    torch.cuda.synchronize()
    lgh = host(lg)
    ids, _ = moe.router(lgh, k, cfg["norm"])
    assert (host(B.ids).astype(np.uint32) == ids).all()
    c, o, od, iv = moe.group_rows(ids.reshape(-1), E)
    assert (host(B.G.offsets).astype(np.uint32) == o).all()
    assert (host(B.G.order).astype(np.uint32) == od).all()
    assert (host(B.G.inv).astype(np.uint32) == iv).all()
    rng = np.random.default_rng(0)
    sample = np.sort(rng.choice(T, 48, replace=False))
    sample[0] = 0
    sample[-1] = T - 1
    xs = host(x.float())[sample]
    _, _, want = moe.layer(xs, lgh[sample], tuple(host(b) for b in (L.wg, L.wu, L.wd)), cfg["types"], k,
                           cfg["norm"])
    got = host(out.float())[sample]
    # the output is bf16: held to the oracle rounded to bf16 the same way, at the north-star bar
    want_bf16 = host(torch.from_numpy(want.astype(np.float32)).to(torch.bfloat16).float())
    assert moe.rel_l2(got, want_bf16) < BAR
    assert rows_ok(got, want_bf16) < ROW_BAR
    assert np.isfinite(host(out.float())).all()



def test_prefill_stack_layer_major():
    """PrefillStack: 3 layers, each layer's output against the oracle on the GPU's own input to that layer (and its
    router logits, so near-ties pick the same experts), the residual fused."""
    from larder_amd import grouped, workloads
    cfg = dict(workloads.CONFIGS[2], E=32)
    g = torch.Generator(device="cuda").manual_seed(21)
    layers = [workloads.make_layer(cfg, g) for _ in range(3)]
    T = 200
    S = grouped.PrefillStack(layers, T, dtype=torch.float32)
    x = torch.randn((T, cfg["H"]), generator=g, device="cuda")
    out, trace = S.run(x, keep=True)
    torch.cuda.synchronize()
    outs = [t[0] for t in trace[1:]] + [out]
    for L, (xin, lg), xo in zip(layers, trace, outs):
        xs = host(xin.half().float())
        _, _, want = moe.layer(xs, host(lg), tuple(host(b) for b in (L.wg, L.wu, L.wd)), cfg["types"], cfg["k"],
                               cfg["norm"], residual=host(xin))
        xr = host(xin)
        assert moe.rel_l2(host(xo) - xr, want - xr) < BAR


@pytest.mark.parametrize("t,bm,ks", [("Q4_0", 32, 1), ("Q4_0", 64, 1), ("Q4_0", 128, 1), ("Q4_0", 32, 4),
                                     ("Q4_0", 32, 2), ("Q4_K", 32, 1), ("Q4_K", 64, 1), ("Q4_K", 128, 1)])
def test_q4_0_tile_rows_both_kernels(t, bm, ks):
    """The Q4_0 GEMMs at both tile heights (32 rows with five K steps in flight, 128 with three), split-K over
    32-row tiles (4 and 2 slices), and the Q4_K GEMMs at both heights (32 rows with three steps prefetched in
    registers), on the same ragged rows, gate/up and down, against the oracle: groups of 0, 1, 31, 32, 33, 64 and
    200 rows, a slot past the experts."""
    from larder_amd import grouped
    types, H, I, E = (t,) * 3, 2048, 768, 9
    w = experts(types, H, I, E, 77)
    rng = np.random.default_rng(bm)
    sizes = [0, 1, 31, 32, 33, 64, 200, 5, 2]
    slots = np.concatenate([np.full(n, e) for e, n in enumerate(sizes)]).astype(np.int32)
    rng.shuffle(slots)
    slots[3] = E + 1
    R = slots.size
    x = dev(rng.standard_normal((R, H)).astype(np.float16))
    G = grouped.Grouping(R, E, bm=bm).run(dev(slots))
    h = torch.empty((R, I), dtype=torch.float16, device="cuda")
    y = torch.empty((R, H), dtype=torch.float32, device="cuda")
    grouped.gate_up(x, G, 1, dev(w[0]), dev(w[1]), types, h, ksplit=ks)
    grouped.down(h, G, dev(w[2]), types[2], y, ksplit=ks)
    torch.cuda.synchronize()
    order = host(G.order)
    valid = slots[order] < E
    hw, yw = moe.gemv(host(x.float()), w, slots, 1, types)
    got_h = host(grouped.from_kperm(h).float())[valid]
    assert moe.rel_l2(got_h, hw[order][valid]) < BAR
    got_y = host(y)[valid]
    assert moe.rel_l2(got_y, yw[order][valid]) < BAR
    assert rows_ok(got_y, yw[order][valid]) < ROW_BAR



@pytest.mark.parametrize("H,I,E,ks", [(2048, 768, 9, 1), (2048, 768, 9, 2), (4096, 1408, 7, 2), (2048, 1408, 9, 1),
                                      (512, 640, 5, 1), (2048, 768, 9, 4)])
def test_q4_0_two_unit_steps_same_bits(H, I, E, ks, monkeypatch):
    """The 32-row Q4_0 GEMMs on the GGUF layout take two units (K 128) a step where the slices' K steps pair up,
    over 2 LDS stages (default) or 3 (LMOE_Q0_W2=3); else, or with LMOE_Q0_W2=1, the one-unit kernel runs: h and
    y bit-equal to the one-unit kernel's, gate/up and down, with and without split-K, on groups of 0, 1, 31, 32,
    33, 64 and 200 rows and a slot past the experts."""
    from larder_amd import grouped
    types = ("Q4_0",) * 3
    w = tuple(dev(b) for b in experts(types, H, I, E, 91))
    rng = np.random.default_rng(H + I + ks)
    sizes = [0, 1, 31, 32, 33, 64, 200, 5, 2][:E]
    slots = np.concatenate([np.full(n, e) for e, n in enumerate(sizes)]).astype(np.int32)
    rng.shuffle(slots)
    slots[3] = E + 1
    R = slots.size
    x = dev(rng.standard_normal((R, H)).astype(np.float16))
    G = grouped.Grouping(R, E, bm=32).run(dev(slots))
    outs = []
    for knob in ("1", "", "3"):
        monkeypatch.setenv("LMOE_Q0_W2", knob)
        h = torch.empty((R, I), dtype=torch.float16, device="cuda")
        y = torch.empty((R, H), dtype=torch.float32, device="cuda")
        grouped.gate_up(x, G, 1, w[0], w[1], types, h, ksplit=ks)
        grouped.down(h, G, w[2], types[2], y, ksplit=ks)
        torch.cuda.synchronize()
        outs.append((host(h), host(y)))
    order = host(G.order)
    valid = slots[order] < E
    h0, y0 = outs[0]
    for h1, y1 in outs[1:]:
        assert np.array_equal(h0.view(np.uint16)[valid], h1.view(np.uint16)[valid])
        assert np.array_equal(y0.view(np.uint32)[valid], y1.view(np.uint32)[valid])
    _, yw = moe.gemv(host(x.float()), tuple(host(b) for b in w), slots, 1, types)
    assert moe.rel_l2(y1[valid], yw[order][valid]) < BAR


@pytest.mark.parametrize("H,I,E", [(1024, 512, 9), (2048, 768, 7), (4096, 256, 5), (512, 1536, 9)])
def test_q4_k_pair_staging_same_bits(H, I, E, monkeypatch):
    """The 64-row Q4_K GEMMs on the GGUF layout with the weights staged two steps at a time (the default): h and y
    bit-equal to the one-step kernel's (LMOE_QK_W2=1), gate/up and down, on groups of 0, 1, 31, 32, 33, 64 and 200 rows and a slot
    past the experts; K from one super-block (down at I = 256) up."""
    from larder_amd import grouped
    types = ("Q4_K",) * 3
    w = tuple(dev(b) for b in experts(types, H, I, E, 93))
    rng = np.random.default_rng(H + 3 * I)
    sizes = [0, 1, 31, 32, 33, 64, 200, 5, 2][:E]
    slots = np.concatenate([np.full(n, e) for e, n in enumerate(sizes)]).astype(np.int32)
    rng.shuffle(slots)
    slots[3] = E + 1
    R = slots.size
    x = dev(rng.standard_normal((R, H)).astype(np.float16))
    G = grouped.Grouping(R, E, bm=64).run(dev(slots))
    outs = []
    for knob in ("1", ""):
        monkeypatch.setenv("LMOE_QK_W2", knob)
        h = torch.empty((R, I), dtype=torch.float16, device="cuda")
        y = torch.empty((R, H), dtype=torch.float32, device="cuda")
        grouped.gate_up(x, G, 1, w[0], w[1], types, h)
        grouped.down(h, G, w[2], types[2], y)
        torch.cuda.synchronize()
        outs.append((host(h), host(y)))
    order = host(G.order)
    valid = slots[order] < E
    (h0, y0), (h1, y1) = outs
    assert np.array_equal(h0.view(np.uint16)[valid], h1.view(np.uint16)[valid])
    assert np.array_equal(y0.view(np.uint32)[valid], y1.view(np.uint32)[valid])
    _, yw = moe.gemv(host(x.float()), tuple(host(b) for b in w), slots, 1, types)
    assert moe.rel_l2(y1[valid], yw[order][valid]) < BAR


@pytest.mark.parametrize("bm,H,I,E", [(128, 2048, 768, 9), (64, 2048, 768, 9), (128, 512, 1408, 5), (128, 256, 128, 4)])
def test_q4_0_tall_pair_staging_same_bits(bm, H, I, E, monkeypatch):
    """The 128- and 64-row Q4_0 GEMMs on the GGUF layout with the weights staged two units at a time (the
    default): h and y bit-equal to the one-unit kernel's (LMOE_Q0_P2=1), gate/up and down, on groups of 0, 1, 31, 32, 33, 64
    and 200 rows and a slot past the experts; K from two units (down at I = 128) up."""
    from larder_amd import grouped
    types = ("Q4_0",) * 3
    w = tuple(dev(b) for b in experts(types, H, I, E, 95))
    rng = np.random.default_rng(bm + H + I)
    sizes = [0, 1, 31, 32, 33, 64, 200, 5, 2][:E]
    slots = np.concatenate([np.full(n, e) for e, n in enumerate(sizes)]).astype(np.int32)
    rng.shuffle(slots)
    slots[3] = E + 1
    R = slots.size
    x = dev(rng.standard_normal((R, H)).astype(np.float16))
    G = grouped.Grouping(R, E, bm=bm).run(dev(slots))
    outs = []
    for knob in ("1", ""):
        monkeypatch.setenv("LMOE_Q0_P2", knob)
        h = torch.empty((R, I), dtype=torch.float16, device="cuda")
        y = torch.empty((R, H), dtype=torch.float32, device="cuda")
        grouped.gate_up(x, G, 1, w[0], w[1], types, h, ksplit=1)
        grouped.down(h, G, w[2], types[2], y, ksplit=1)
        torch.cuda.synchronize()
        outs.append((host(h), host(y)))
    order = host(G.order)
    valid = slots[order] < E
    (h0, y0), (h1, y1) = outs
    assert np.array_equal(h0.view(np.uint16)[valid], h1.view(np.uint16)[valid])
    assert np.array_equal(y0.view(np.uint32)[valid], y1.view(np.uint32)[valid])
    _, yw = moe.gemv(host(x.float()), tuple(host(b) for b in w), slots, 1, types)
    assert moe.rel_l2(y1[valid], yw[order][valid]) < BAR
