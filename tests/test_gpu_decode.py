"""GPU parity of the decode path against the CPU oracle, through the C ABI (larder_amd wrappers).

Bars: expert ids and groupings bit-exact, ties to the lowest expert index; layer
outputs within 2e-3 relative L2 of an fp32 dequant-then-matmul. Quantizer and dequant are integer/byte work and
must be bit-exact."""
import numpy as np
import pytest
import torch

from oracle import gguf, moe

pytestmark = pytest.mark.gpu

BAR = 2e-3


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.detach().cpu().numpy()


def tie_logits(rng, T, E):
    lg = rng.normal(0, 1.0, (T, E)).astype(np.float32) * rng.uniform(0.5, 4.0)
    for r in range(T):
        if r % 5 == 0:
            j = rng.integers(0, E, 6)
            lg[r, j] = lg[r, j[0]]
        if r % 7 == 0:
            lg[r] = np.round(lg[r] * 2) / 2
        if r % 13 == 0:
            lg[r] = 0.25
    return lg


@pytest.mark.parametrize("E,k,norm", [(60, 4, False), (128, 8, True), (512, 10, True), (1024, 32, False), (9, 9, True)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_router_topk_bit_exact(E, k, norm, dtype):
    from larder_amd import route
    rng = np.random.default_rng(E * 7 + k)
    # tie-heavy rows, then all-negative rows in steps of 0.5 (the k-th key negative and tied)
    neg = (-np.round(np.abs(rng.normal(0, 2.0, (16, E))) * 2) / 2 - 0.5).astype(np.float32)
    lg = np.concatenate([tie_logits(rng, 67, E), neg])
    x = dev(lg).to(dtype)
    ids, sc = route.topk(x, k, norm)
    lg32 = host(x.float())
    want_ids, want_sc = moe.router(lg32, k, norm)
    assert (host(ids).astype(np.uint32) == want_ids).all()
    assert np.allclose(host(sc), want_sc, rtol=2e-6, atol=1e-7)
    inds, sc2 = route.probs(x, k, norm)
    assert (host(inds)[:, ::-1].astype(np.uint32) == want_ids).all()


def test_quantize_q4_0_bit_exact():
    from larder_amd import _lib
    rng = np.random.default_rng(11)
    w = rng.standard_normal((300, 256)).astype(np.float32) * 0.02
    w[0] = 0.0
    w[1, :32] = np.float32(0.5)
    w[1, 7] = -0.5                 # equal magnitudes: the first one sets the sign of d
    w[2, :32] = (np.arange(32) - 16) / 4.0
    w[3, 5] = 1e-30
    for dt in (torch.float32, torch.float16, torch.bfloat16):
        wt = dev(w).to(dt)
        out = torch.empty((300, 256 // 32 * 18), dtype=torch.uint8, device="cuda")
        _lib.call("lmoe_quantize_q4_0", _lib.ptr(wt), _lib.dcode(dt), 300, 256, _lib.ptr(out), _lib.stream())
        want = gguf.quantize_q4_0(host(wt.float()))
        assert (host(out) == want).all(), dt


@pytest.mark.parametrize("t", ["Q4_0", "Q4_K"])
@pytest.mark.parametrize("odt", [torch.float32, torch.float16])
def test_dequant(t, odt):
    from larder_amd import gguf_experts as ge
    rng = np.random.default_rng(12)
    buf = gguf.random_experts(rng, 5, 16, 512, t)
    slots = np.array([3, 0, 9, 4], np.int32)          # 9: no such expert -> zeros
    q = ge.dequant(dev(buf), dev(slots), t, odt)
    want = np.zeros((4, 16, 512), np.float32)
    for i, s in enumerate(slots):
        if s < 5:
            want[i] = gguf.dequant_matrix(buf[s], t)
    got = host(q.float())
    if odt == torch.float32:
        assert (got.view(np.uint32) == want.view(np.uint32)).all()
    else:
        assert (got == want.astype(np.float16).astype(np.float32)).all()


MIXES = [(("Q4_0",) * 3, 2048, 768), (("Q4_0",) * 3, 2048, 1408), (("Q4_0",) * 3, 512, 256),
         (("Q4_0",) * 3, 1344, 448), (("Q4_K",) * 3, 1024, 512), (("Q4_K",) * 3, 4096, 256),
         (("Q4_0", "Q4_K", "Q4_0"), 1024, 512), (("Q4_K", "Q4_0", "Q4_K"), 512, 512)]


@pytest.mark.parametrize("types,H,I", MIXES)
@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16, torch.float32])
def test_gemv_chain_vs_oracle(types, H, I, xdt):
    from larder_amd import gguf_experts as ge
    rng = np.random.default_rng(H + I)
    E = 6
    w = tuple(gguf.random_experts(rng, E, r, c, t) for (r, c), t in zip(((I, H), (I, H), (H, I)), types))
    topk, rows = 2, 3
    slots = rng.integers(0, E, rows * topk).astype(np.int32)
    slots[-1] = E + 3                                    # no such expert: zero rows
    x = dev(rng.standard_normal((rows, H)).astype(np.float32)).to(xdt)
    h, y = ge._chain(x, tuple(dev(b) for b in w), dev(slots), topk, types, torch.float32)
    # the kernels see x as f16; feed the oracle the same values
    xs = host(x.float().half().float())
    hw, yw = moe.gemv(xs, w, slots, topk, types)
    assert (host(h)[-1] == 0).all() and (host(y)[-1] == 0).all()
    assert moe.rel_l2(host(h), hw) < 1e-5
    assert moe.rel_l2(host(y), yw) < BAR
    y16 = ge.gemv(x, tuple(dev(b) for b in w), dev(slots), topk, "/".join(types), torch.float16)
    assert moe.rel_l2(host(y16.float()), yw) < BAR


@pytest.mark.parametrize("t,H,I", [("Q4_0", 2048, 768), ("Q4_K", 4096, 512), ("Q4_0", 4096, 512),
                                   ("Q4_K", 2048, 768), ("Q4_0", 2048, 1408)])
def test_gate_up_prepped_vs_oracle(t, H, I):
    """lmoe_gemv_gate_up_prepped (activations prepared once, the register-resident kernel at H = 2048 / 4096) with
    f32 h and with prepared h, slots in no particular order and one past the experts."""
    from larder_amd._lib import call, dcode, ptr, qcode, stream
    rng = np.random.default_rng(H * 3 + I)
    E, T, topk = 5, 2, 3
    wg = gguf.random_experts(rng, E, I, H, t)
    wu = gguf.random_experts(rng, E, I, H, t)
    x = dev(rng.standard_normal((T, H)).astype(np.float32)).half()
    xprep = torch.empty((T, H // 64 * 36), dtype=torch.int32, device="cuda")
    call("lmoe_prep_x", ptr(x), dcode(x.dtype), T, H, qcode(t), ptr(xprep), stream())
    slots = np.array([3, 0, 4, 1, E + 2, 2], np.int32)
    h = torch.full((T * topk, I), 7.0, dtype=torch.float32, device="cuda")
    hp = torch.zeros((T * topk, I // 64 * 36), dtype=torch.int32, device="cuda")
    sd, wgd, wud = dev(slots), dev(wg), dev(wu)  # held until the kernel has run
    call("lmoe_gemv_gate_up_prepped", ptr(xprep), ptr(xprep), ptr(sd), T * topk, topk, ptr(wgd), ptr(wud), qcode(t),
         qcode(t), E, H, I, ptr(h), ptr(hp), qcode(t), stream())
    torch.cuda.synchronize()
    xs = host(x.float())
    hw, _ = moe.gemv(xs, (wg, wu, gguf.random_experts(rng, E, H, I, t)), slots, topk, (t, t, t))
    got = host(h)
    assert (got[4] == 0).all()
    assert moe.rel_l2(got, hw) < 1e-5
    # the prepared copy holds the same values as f16, at the unit dword / half the layout gives each element
    hs = 32 if t == "Q4_K" else 16
    halves = host(hp).view(np.float16).reshape(T * topk, I // 64, 72)
    for e in (0, 1, 63, I - 1):
        span, f = divmod(e % 64, 2 * hs)
        hi, g = divmod(f, hs)
        dw = span * hs + 4 * (g >> 2) + 2 * ((g & 3) & 1) + hi
        half = (g & 3) >> 1
        assert (halves[:, e // 64, 2 * dw + half].astype(np.float32) == got[:, e].astype(np.float16)).all()


@pytest.mark.parametrize("T,k,E,H,I", [(1, 8, 16, 2048, 768), (3, 4, 10, 1024, 1408), (5, 10, 12, 512, 512)])
def test_down_combine_vs_oracle(T, k, E, H, I):
    from larder_amd import _lib
    rng = np.random.default_rng(T * 100 + k)
    wd = gguf.random_experts(rng, E, H, I, "Q4_0")
    h = rng.standard_normal((T * k, I)).astype(np.float32)
    ids = rng.integers(0, E, (T, k)).astype(np.int32)
    sc = rng.uniform(0, 1, (T, k)).astype(np.float32)
    shared = rng.standard_normal((T, H)).astype(np.float32)
    gate = rng.standard_normal((T, 3)).astype(np.float32)
    res = rng.standard_normal((T, H)).astype(np.float16)
    out = torch.empty((T, H), dtype=torch.float32, device="cuda")
    hd, idd, scd, shd, gd, rd, wdd = dev(h), dev(ids), dev(sc), dev(shared), dev(gate), dev(res), dev(wd)
    _lib.call("lmoe_gemv_down_combine", _lib.ptr(hd), _lib.ptr(idd), _lib.ptr(scd), T, k, _lib.ptr(wdd),
              _lib.Q4_0, E, I, H, _lib.ptr(shd), _lib.ptr(gd), 3, _lib.ptr(rd), _lib.F16, _lib.ptr(out), _lib.F32,
              _lib.stream())
    wdf = gguf.dequant_matrix(wd, "Q4_0")
    h16 = h.astype(np.float16).astype(np.float32)            # h meets the weights as f16
    y = np.einsum("tki,tkhi->tkh", h16.reshape(T, k, I), wdf[ids])
    want = moe.combine(y, sc, shared, gate[:, 0], res.astype(np.float32))
    assert moe.rel_l2(host(out), want) < 1e-5


def _layer_from_device(cfg, seed):
    from larder_amd import workloads
    g = torch.Generator(device="cuda").manual_seed(seed)
    return workloads.make_layer(cfg, g)


@pytest.mark.parametrize("T", [1, 3])
def test_decode_layer_cfg1_vs_oracle(T):
    """Config 1's layer (E 60, top-4, no renorm, I 1408, shared 5632 + sigmoid gate) at T tokens."""
    from larder_amd import layer as lay, workloads
    cfg = workloads.CONFIGS[1]
    L = _layer_from_device(cfg, 0)
    rng = np.random.default_rng(T)
    x = dev(rng.standard_normal((T, cfg["H"])).astype(np.float16))
    B = lay.DecodeBuffers(L, T)
    out = torch.empty((T, cfg["H"]), dtype=torch.float32, device="cuda")
    lay.decode(L, x, B, out)
    torch.cuda.synchronize()
    xs = host(x.float())
    lg_gpu = host(B.logits)
    # routing pinned from x: the router GEMV's fixed order restated bit for bit, ids from the oracle's own logits
    lg_ref = moe.router_logits_gemv(host(x), host(L.wr))
    assert np.array_equal(lg_gpu[:, :cfg["E"]].view(np.uint32), lg_ref.view(np.uint32))
    gate_ref = moe.router_logits_gemv(host(x), host(L.wsg).reshape(1, -1))
    assert np.array_equal(lg_gpu[:, cfg["E"]:].view(np.uint32), gate_ref.view(np.uint32))
    ids, _, want = moe.layer(xs, lg_ref, tuple(host(b) for b in (L.wg, L.wu, L.wd)), cfg["types"],
                             cfg["k"], cfg["norm"], shared=tuple(host(b[0]) for b in L.shared),
                             shared_gate_w=host(L.wsg.float()))
    assert (host(B.ids).astype(np.uint32) == ids).all()
    assert moe.rel_l2(host(out), want) < BAR


@pytest.mark.parametrize("T", [1, 3])
def test_cfg1_shared_slices_folded_match_apart(T):
    """Config 1's 5,632-wide shared expert folded into the decode kernels as four slices of the routed width (slots
    k .. k + 3, ids E .. E + 3, each weighted by the gate's sigmoid: three launches a layer) against the same layer
    with the shared expert run apart (five launches): equal ids, outputs within the bar of each other and of the
    oracle."""
    from larder_amd import layer as lay, workloads
    cfg = workloads.CONFIGS[1]
    L = _layer_from_device(cfg, 12)
    assert L.folded is not None and L.n_shared == 4
    U = lay.MoELayer(L.wg, L.wu, L.wd, L.types, L.k, L.norm, wr=L.wr, shared=L.shared, wsg=L.wsg,
                     fold_shared=False)
    assert U.folded is None
    rng = np.random.default_rng(T + 40)
    x = dev(rng.standard_normal((T, cfg["H"])).astype(np.float16))
    outs = []
    for layer in (L, U):
        B = lay.DecodeBuffers(layer, T)
        out = torch.empty((T, cfg["H"]), dtype=torch.float32, device="cuda")
        lay.decode(layer, x, B, out)
        torch.cuda.synchronize()
        outs.append((host(out), host(B.ids).copy(), B))
    (of, idf, Bf), (ou, idu, _) = outs
    assert (idf == idu).all()
    lg = host(Bf.logits)
    assert (host(Bf.ids_ext)[:, cfg["k"]:] == cfg["E"] + np.arange(4)).all()
    assert np.allclose(host(Bf.scores_ext)[:, cfg["k"]:], 1 / (1 + np.exp(-lg[:, cfg["E"]:cfg["E"] + 1])), rtol=1e-5)
    assert moe.rel_l2(of, ou) < BAR
    _, _, want = moe.layer(host(x.float()), lg[:, :cfg["E"]], tuple(host(b) for b in (L.wg, L.wu, L.wd)),
                           cfg["types"], cfg["k"], cfg["norm"], shared=tuple(host(b[0]) for b in L.shared),
                           shared_gate_w=host(L.wsg.float()))
    assert moe.rel_l2(of, want) < BAR


def test_decode_layer_cfg2_residual():
    from larder_amd import layer as lay, workloads
    cfg = workloads.CONFIGS[2]
    L = _layer_from_device(cfg, 1)
    rng = np.random.default_rng(9)
    x = dev(rng.standard_normal((1, cfg["H"])).astype(np.float16))
    B = lay.DecodeBuffers(L, 1)
    out = torch.empty((1, cfg["H"]), dtype=torch.float32, device="cuda")
    lay.decode(L, x, B, out, residual=x)
    torch.cuda.synchronize()
    xs = host(x.float())
    lg = moe.router_logits_gemv(host(x), host(L.wr))  # routing pinned from x, bit for bit
    assert np.array_equal(host(B.logits).view(np.uint32), lg.view(np.uint32))
    ids, _, want = moe.layer(xs, lg, tuple(host(b) for b in (L.wg, L.wu, L.wd)), cfg["types"], cfg["k"],
                             cfg["norm"], residual=xs)
    assert (host(B.ids).astype(np.uint32) == ids).all()
    assert moe.rel_l2(host(out.float()) - xs, want - xs) < BAR


def test_graph_replay_matches_eager():
    """A captured 3-layer step replays to the eager result, bit for bit, with eager work between replays."""
    from larder_amd import layer as lay, workloads
    cfg = dict(workloads.CONFIGS[2], E=16)
    g = torch.Generator(device="cuda").manual_seed(5)
    layers = [workloads.make_layer(cfg, g) for _ in range(3)]
    st = lay.DecodeStack(layers, 1)
    xs = torch.randn((4, 1, cfg["H"]), generator=g, device="cuda").half()
    eager = []
    for i in range(4):
        st.x_in.copy_(xs[i])
        eager.append(st.step().clone())
    graph = st.capture()
    for i in range(4):
        st.x_in.copy_(xs[i])
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(st.x_out, eager[i]), i
        _ = torch.randn(1000, device="cuda").sum().item()     # eager work and a sync between replays


@pytest.mark.parametrize("R,E,bm", [(1, 4, 16), (8, 128, 16), (512, 128, 32), (65536, 128, 128), (5000, 60, 64),
                                    (3000, 1024, 16),
                                    # one workgroup (R <= 1024): the E = 1024 edge (ids past it in bucket 1024), a
                                    # handful of experts, one expert, and the first size past it
                                    (1024, 1024, 16), (777, 1024, 32), (1024, 3, 128), (64, 1, 16), (1025, 60, 32)])
def test_group_rows_bit_exact(R, E, bm):
    from larder_amd import _lib
    rng = np.random.default_rng(R + E)
    ids = rng.integers(0, E, R).astype(np.int32)
    if R > 10:
        ids[rng.integers(0, R, R // 50)] = E + 5            # rows with no such expert go last
        ids[: R // 3] = rng.integers(0, 3, R // 3)          # skew: a few experts take many rows
    d = dev(ids)
    counts = torch.empty(E, dtype=torch.int32, device="cuda")
    offsets = torch.empty(E + 1, dtype=torch.int32, device="cuda")
    order = torch.empty(R, dtype=torch.int32, device="cuda")
    inv = torch.empty(R, dtype=torch.int32, device="cuda")
    mt = _lib.lib().lmoe_max_tiles(R, E, bm)
    tiles = torch.empty(mt, dtype=torch.int32, device="cuda")
    nt = torch.empty(1, dtype=torch.int32, device="cuda")
    ws = torch.empty(_lib.lib().lmoe_group_workspace_bytes(R, E) // 4 + 1, dtype=torch.int32, device="cuda")
    _lib.call("lmoe_group_rows", _lib.ptr(d), R, E, bm, _lib.ptr(counts), _lib.ptr(offsets), _lib.ptr(order),
              _lib.ptr(inv), _lib.ptr(tiles), _lib.ptr(nt), _lib.ptr(ws), _lib.stream())
    c, o, od, iv = moe.group_rows(ids.astype(np.uint32), E)
    assert (host(counts).astype(np.uint32) == c).all()
    assert (host(offsets).astype(np.uint32) == o).all()
    assert (host(order).astype(np.uint32) == od).all()
    assert (host(inv).astype(np.uint32) == iv).all()
    n = int(host(nt)[0])
    want = [(e << 20) | m for e in range(E) for m in range(-(-int(c[e]) // bm))]
    assert n == len(want) <= mt and host(tiles)[:n].tolist() == want


def test_tail_combine_vs_oracle():
    from larder_amd import route
    rng = np.random.default_rng(21)
    T, k, D = 5, 8, 2048
    y = rng.standard_normal((1, T, k, D)).astype(np.float32)
    sc = rng.uniform(0, 1, (1, T, k)).astype(np.float32)
    sh = rng.standard_normal((1, T, D)).astype(np.float32)
    gt = rng.standard_normal((1, T, 1)).astype(np.float32)
    got = route.tail(dev(y), dev(sc), dev(sh), dev(gt))
    want = moe.combine(y[0], sc[0], sh[0], gt[0, :, 0])
    assert moe.rel_l2(host(got)[0], want) < 1e-6


@pytest.mark.parametrize("E,k,norm,T,shared,H", [(60, 4, False, 1, 1, 2048), (128, 8, True, 1, 0, 2048),
                                                  (128, 8, True, 5, 0, 2048), (512, 10, True, 1, 1, 4096),
                                                  (512, 16, False, 3, 0, 2048), (9, 9, True, 2, 0, 2048),
                                                  (256, 8, True, 16, 1, 4096), (129, 7, True, 4, 0, 2048),
                                                  (60, 4, False, 3, 4, 2048)])
def test_router_gemv_rank_vs_oracle(E, k, norm, T, shared, H):
    """lmoe_router_gemv_rank (GEMV + top-k in one launch, the last workgroup ranking): logits bit-exact against the
    router GEMV's restated order, ids bit-exact against the oracle's top-k of those logits (planted equal rows: ties
    to the lowest index), scores to 2e-6, the folded shared expert's slot, and a second launch on the same arrival
    counter giving the same bits. shared: the folded shared expert's slices a token (0: none)."""
    from larder_amd import _lib
    rng = np.random.default_rng(E * 31 + k * 7 + T)
    wr = (rng.standard_normal((E, H)) * 0.02).astype(np.float16)
    for grp in (rng.choice(E, min(4, E), replace=False), rng.choice(E, min(3, E), replace=False)):
        wr[grp] = wr[grp[0]] * np.float16(3)              # equal rows: exactly equal logits
    x = rng.standard_normal((T, H)).astype(np.float16)
    wsg = (rng.standard_normal(H) * 0.02).astype(np.float16) if shared else None
    ks = k + shared
    rows = E + (1 if shared else 0)
    dx, dwr = dev(x), dev(wr)
    dwsg = dev(wsg) if shared else None
    sync = torch.zeros(1, dtype=torch.int32, device="cuda")
    outs = []
    for _ in range(2):
        lg = torch.full((T, rows), float("nan"), device="cuda")
        ids = torch.full((T, ks), -1, dtype=torch.int32, device="cuda")
        sc = torch.full((T, ks), float("nan"), device="cuda")
        xp = torch.empty((T, H // 64 * 36), dtype=torch.int32, device="cuda")
        _lib.call("lmoe_router_gemv_rank", _lib.ptr(dx), _lib.F16, _lib.ptr(dwr), _lib.ptr(dwsg), _lib.F16, T, H, E, k,
                  int(norm), ks, _lib.ptr(lg), _lib.ptr(ids), _lib.ptr(sc), _lib.ptr(xp), _lib.Q4_0, _lib.ptr(sync),
                  _lib.stream())
        torch.cuda.synchronize()
        outs.append((host(lg), host(ids), host(sc)))
    assert int(sync.item()) == 0
    lg, ids, sc = outs[0]
    for a, b in zip(outs[0], outs[1]):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    want_lg = moe.router_logits_gemv(x, wr)
    assert np.array_equal(lg[:, :E].view(np.uint32), want_lg.view(np.uint32))
    want_ids, want_sc = moe.router(want_lg, k, norm)
    assert (ids[:, :k].astype(np.uint32) == want_ids).all()
    assert np.allclose(sc[:, :k], want_sc, rtol=2e-6, atol=1e-7)
    if shared:
        gate = moe.router_logits_gemv(x, wsg.reshape(1, -1))
        assert np.array_equal(lg[:, E:].view(np.uint32), gate.view(np.uint32))
        assert (ids[:, k:] == E + np.arange(shared)).all()
        assert np.allclose(sc[:, k:], moe.sigmoid(gate[:, :1]), rtol=1e-6)


@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float32])
def test_decode_f16_range_limit(xdt):
    """The decode chain's stated limit: x and h meet the weights as f16 (the reference stages both as f32,
    gguf_experts.py:452-526). Inside f16's range the layer and the drop-in gemv hold the bar; an |x| past 65,504
    (bf16 / f32 x) or an |h| past it (x inside the range, weights large enough) makes the rows it feeds non-finite,
    while the router, which reads x as given, still routes as the oracle does."""
    from larder_amd import gguf_experts as ge, layer as lay, workloads
    cfg = dict(workloads.CONFIGS[2], E=16)
    L = _layer_from_device(cfg, 4)
    rng = np.random.default_rng(17)
    H = cfg["H"]
    w = tuple(host(b) for b in (L.wg, L.wu, L.wd))
    base = rng.standard_normal((2, H)).astype(np.float32)
    cases = {"inside": base * 8.0, "x_past_f16": base.copy(), "h_past_f16": base * 300.0}
    cases["x_past_f16"][:, ::97] = 1.0e5
    for name, xa in cases.items():
        x = dev(xa).to(xdt)
        xs = host(x.float())
        B = lay.DecodeBuffers(L, 2)
        out = torch.empty((2, H), dtype=torch.float32, device="cuda")
        lay.decode(L, x, B, out)
        torch.cuda.synchronize()
        if xdt == torch.bfloat16:  # routing pinned from x (bf16 x widened exactly; every product exact in fp32)
            lg = moe.router_logits_gemv(xs, host(L.wr))
            assert np.array_equal(host(B.logits).view(np.uint32), lg.view(np.uint32)), name
        else:  # f32 x: the router's fma products round, which the oracle's order does not restate; its ids from them
            lg = host(B.logits)
        ids, _, want = moe.layer(xs, lg, w, cfg["types"], cfg["k"], cfg["norm"])
        assert (host(B.ids).astype(np.uint32) == ids).all(), name
        slots = torch.from_numpy(ids.reshape(-1).astype(np.int32)).cuda()
        y = host(ge.gemv(x, (L.wg, L.wu, L.wd), slots, cfg["k"], cfg["types"], torch.float32))
        hw, yw = moe.gemv(xs, w, ids.reshape(-1), cfg["k"], cfg["types"])
        if name == "inside":
            assert np.abs(hw).max() < 65504 and moe.rel_l2(host(out), want) < BAR and moe.rel_l2(y, yw) < BAR
        else:
            if name == "h_past_f16":  # the premise: x inside f16's range, h past it
                assert np.abs(xs).max() < 65504 and np.abs(hw).max() > 65504
            assert not np.isfinite(host(out)).all() and not np.isfinite(y).all(), name
