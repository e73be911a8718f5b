"""The decode layer's gate/up and down in one launch (lmoe_moe_fused) against the two-launch chain
(lmoe_moe_gate_up[_ext] + lmoe_gemv_down_combine_prepped), bit for bit, and against the oracle; repeated launches
over one workspace (the per-workgroup epochs), graph replay, and the refusals.

The chain is the reference's decode order (gguf_experts.py:452-526 over route_cuda.probs, route_cuda.py:433-444),
already pinned to the oracle by test_gpu_decode.py; the one-launch form must give its ids, scores and outputs bit for
bit.
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
    return workloads.make_layer(cfg, g)


SHAPES = {
    "cfg2": dict(H=2048, E=128, k=8, I=768, norm=True, Is=0, types=("Q4_0",) * 3),
    "q4k_2048": dict(H=2048, E=64, k=6, I=512, norm=True, Is=0, types=("Q4_K",) * 3),
    "q40_h4096": dict(H=4096, E=32, k=4, I=768, norm=False, Is=0, types=("Q4_0",) * 3),
    "cfg5": dict(H=4096, E=512, k=10, I=512, norm=True, Is=512, types=("Q4_K",) * 3),
    "folded2_q40": dict(H=2048, E=60, k=4, I=512, norm=False, Is=1024, types=("Q4_0",) * 3),
    # two h units a down lane on Q4_K, E 512 on Q4_0, and cfg5's shape without its shared expert
    "q4k_nu2": dict(H=2048, E=64, k=8, I=1024, norm=True, Is=0, types=("Q4_K",) * 3),
    "q40_e512": dict(H=2048, E=512, k=8, I=768, norm=True, Is=0, types=("Q4_0",) * 3),
    "cfg5_unshared": dict(H=4096, E=512, k=10, I=512, norm=True, Is=0, types=("Q4_K",) * 3),
}


def _run(lay, L, x, B, residual, fused):
    old = lay.FUSED
    lay.FUSED = fused
    try:
        out = torch.empty_like(x, dtype=torch.float32)
        lay.decode(L, x, B, out, residual=residual)
        torch.cuda.synchronize()
        return host(out), host(B.ids_ext).copy(), host(B.scores_ext).copy()
    finally:
        lay.FUSED = old


# cfg5's shape (the largest layer, 1.8 GB of weights) at T 1 and 5 in f16 only; every other shape at every T and dtype
CASES = [(n, T, dt) for n in SHAPES for T in (1, 5, 16) for dt in (torch.float16, torch.bfloat16, torch.float32)
         if n != "cfg5" or (T < 16 and dt == torch.float16)]


@pytest.mark.parametrize("name,T,xdt", CASES)
def test_fused_equals_chain(name, T, xdt):
    """Three calls in a row over one workspace (epochs 1, 2, 3), each with a fresh x, against the chain on the same x:
    ids, scores and outputs bit for bit; with a residual on the second call."""
    from larder_amd import layer as lay
    cfg = SHAPES[name]
    L = _layer(cfg, 3)
    assert lay.fused_ok(L, T)
    B = lay.DecodeBuffers(L, T)
    assert B.fused_ws is not None
    g = torch.Generator(device="cuda").manual_seed(T * 7 + 1)
    for call in range(3):
        x = torch.randn((T, cfg["H"]), generator=g, device="cuda").to(xdt)
        res = x if call == 1 else None
        want = _run(lay, L, x, B, res, False)
        got = _run(lay, L, x, B, res, True)
        assert np.array_equal(got[1], want[1]), (call, "ids")
        assert np.array_equal(got[2].view(np.uint32), want[2].view(np.uint32)), (call, "scores")
        same = got[0].view(np.uint32) == want[0].view(np.uint32)
        assert same.all(), (call, "out", f"status {B.fused_status()}", f"{int((~same).sum())} of {same.size} differ",
                            f"{int(np.isnan(got[0]).sum())} NaN", f"rel {moe.rel_l2(got[0], want[0]):.3g}",
                            f"max {float(np.nanmax(np.abs(got[0] - want[0]))):.3g}")
    assert B.fused_status() == 0


@pytest.mark.parametrize("name", ["cfg2", "cfg5", "folded2_q40"])
def test_fused_vs_oracle(name):
    """Routing pinned from x (the router GEMV's order, restated by the oracle), then ids bit-exact and the layer
    within 2e-3 of the fp32 dequant-then-matmul, on the one-launch path."""
    from larder_amd import layer as lay
    cfg = SHAPES[name]
    L = _layer(cfg, 11)
    T = 2
    rng = np.random.default_rng(5)
    x = torch.from_numpy(rng.standard_normal((T, cfg["H"])).astype(np.float16)).cuda()
    B = lay.DecodeBuffers(L, T)
    out, ids_ext, _ = _run(lay, L, x, B, None, True)
    assert B.fused_status() == 0
    lg = moe.router_logits_gemv(host(x), host(L.wr))
    assert np.array_equal(host(B.logits)[:, :cfg["E"]].view(np.uint32), lg.view(np.uint32))
    shared = sgw = None
    if cfg["Is"]:
        shared = tuple(host(b[0]) for b in L.shared)
        sgw = host(L.wsg.float())
        m = L.n_shared
        assert (ids_ext[:, cfg["k"]:] == cfg["E"] + np.arange(m)).all()
    ids, _, want = moe.layer(host(x.float()), lg, tuple(host(b) for b in (L.wg, L.wu, L.wd)), cfg["types"],
                             cfg["k"], cfg["norm"], shared=shared, shared_gate_w=sgw)
    assert (ids_ext[:, :cfg["k"]].astype(np.uint32) == ids).all()
    assert moe.rel_l2(out, want) < BAR
    for t in range(T):
        assert moe.rel_l2(out[t], want[t]) < 1e-2


def test_fused_graph_replay_matches_eager():
    """A captured 4-layer step on the one-launch path replays to the eager result bit for bit, with eager work and
    synchronisations between replays (every replay is a new epoch of the same workspace)."""
    from larder_amd import layer as lay, workloads
    cfg = dict(workloads.CONFIGS[2], E=32)
    g = torch.Generator(device="cuda").manual_seed(8)
    layers = [workloads.make_layer(cfg, g) for _ in range(4)]
    st = lay.DecodeStack(layers, 1)
    assert st.bufs.fused_ws is not None
    xs = torch.randn((5, 1, cfg["H"]), generator=g, device="cuda").half()
    old = lay.FUSED
    try:
        eager = []
        lay.FUSED = False  # the chain
        for i in range(5):
            st.x_in.copy_(xs[i])
            eager.append(st.step().clone())
        lay.FUSED = True  # the one-launch form, eager: the same bits
        for i in range(5):
            st.x_in.copy_(xs[i])
            assert torch.equal(st.step(), eager[i]), i
        graph = st.capture()  # records the one-launch form
    finally:
        lay.FUSED = old
    for rep in range(3):
        for i in range(5):
            st.x_in.copy_(xs[i])
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(st.x_out, eager[i]), (rep, i)
            _ = torch.randn(1000, device="cuda").sum().item()
    assert st.bufs.fused_status() == 0


def test_fused_refusals():
    """Arguments the one-launch kernel does not take are refused on the host, before any launch."""
    from larder_amd import _lib
    from larder_amd import layer as lay
    cfg = SHAPES["cfg2"]
    L = _layer(cfg, 2)
    B = lay.DecodeBuffers(L, 1)
    x = torch.randn((1, cfg["H"]), device="cuda").half()
    out = torch.empty((1, cfg["H"]), dtype=torch.float32, device="cuda")
    _run(lay, L, x, B, None, True)
    P = _lib.ptr
    q0 = _lib.qcode("Q4_0")
    args = [P(B.logits), B.logits.shape[1], 1, L.k, 1, P(B.xprep), P(L.wg), P(L.wu), P(L.wd), q0, q0, L.E, L.H, L.I,
            0, P(B.ids_ext), P(B.scores_ext), None, None, 0, P(out), _lib.dcode(out.dtype), P(B.fused_ws),
            B.fused_ws.numel() * 4, _lib.stream()]
    short = list(args)
    short[23] = B.fused_ws.numel() * 4 - 8
    with pytest.raises(RuntimeError, match="workspace"):
        _lib.call("lmoe_moe_fused", *short)
    wide = list(args)
    wide[2] = 17
    with pytest.raises(RuntimeError, match="tokens"):
        _lib.call("lmoe_moe_fused", *wide)
    for td in ("Q6_K", "Q4_K"):  # a type beyond Q4, or a down type other than gate/up's
        mixed = list(args)
        mixed[10] = _lib.qcode(td)
        with pytest.raises(ValueError):
            _lib.call("lmoe_moe_fused", *mixed)
    torch.cuda.synchronize()
    assert B.fused_status() == 0
