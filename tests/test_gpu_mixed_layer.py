"""GPU parity of the decode layer (larder_amd.layer.decode, DecodeStack) on layers with a projection beyond
Q4_0 / Q4_K, the route every block type takes in the reference (gguf_experts.py:600-653 over stream_fast.py:4352-4377):
the 35B's Q4_K / Q4_K / Q6_K mix and a Q8_0 down (the prepared chain: gate/up on the register-resident kernel
writing h in the Q4_K / Q4_0 order, the Q6_K / Q8_0 down reading it), a Q5_K down (fp32 h, the general down),
all-Q6_K and Q8_0 gate/up layers (the general gate/up), and given logits.
Routing is pinned from x (the router GEMV's fixed order restated in the oracle, bit for bit) and the outputs are
held to the north star's 2e-3 relative L2 against the fp32 dequant-then-matmul oracle."""
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


def make_layer(rng, types, H, I, E, k, norm, Is=0, router=True, fold=True):
    from larder_amd import layer as lay
    w = [gguf.random_experts(rng, E, r, c, t) for (r, c), t in zip(((I, H), (I, H), (H, I)), types)]
    shared = wsg = None
    if Is:
        shared = tuple(dev(gguf.random_experts(rng, 1, r, c, t))
                       for (r, c), t in zip(((Is, H), (Is, H), (H, Is)), types))
        wsg = dev((rng.standard_normal(H) * 0.02).astype(np.float16))
    wr = dev((rng.standard_normal((E, H)) * 0.02).astype(np.float16)) if router else None
    return lay.MoELayer(*(dev(b) for b in w), types, k, norm, wr=wr, shared=shared, wsg=wsg, fold_shared=fold)


def oracle_out(L, x, residual=None):
    """(ids, out) of the oracle on layer L for x (float16 [T, H] on the device), routing from x in the router
    GEMV's order."""
    xs = host(x.float())
    lg = moe.router_logits_gemv(host(x), host(L.wr))
    shared = tuple(host(b[0]) for b in L.shared) if L.shared is not None else None
    sgw = host(L.wsg.float()) if L.wsg is not None else None
    ids, _, want = moe.layer(xs, lg, tuple(host(b) for b in (L.wg, L.wu, L.wd)), L.types, L.k, L.norm,
                             shared=shared, shared_gate_w=sgw, residual=residual)
    return lg, ids, want


CASES = [
    # (types, H, I, E, k, norm, Is): the 35B's mix without and with a folded shared expert (m = 1 and 2 slices)
    (("Q4_K", "Q4_K", "Q6_K"), 2048, 768, 16, 4, True, 0),
    (("Q4_K", "Q4_K", "Q6_K"), 2048, 512, 12, 4, True, 512),
    (("Q4_K", "Q4_K", "Q6_K"), 4096, 256, 8, 2, False, 512),
    # a Q8_0 down (h prepared in the Q4_0 order) with a shared expert that does not fold (1024 is not a multiple of
    # 768), and with one that folds
    (("Q4_0", "Q4_0", "Q8_0"), 2048, 768, 12, 4, False, 1024),
    (("Q4_0", "Q4_0", "Q8_0"), 4096, 512, 10, 3, True, 1024),
    # a Q5_K down under Q4_K gate/up: fp32 h (lmoe_moe_gate_up_h), the general down; then the same with a folded
    # shared expert (m = 2 slices: lmoe_moe_gate_up_h's sigmoid-weighted slots E, E + 1 and their fp32 h rows)
    (("Q4_K", "Q4_K", "Q5_K"), 2048, 512, 12, 4, True, 0),
    (("Q4_K", "Q4_K", "Q5_K"), 2048, 512, 12, 4, True, 1024),
    # gate/up beyond Q4 (the general gate/up from raw x), down Q6_K or Q4_0
    (("Q6_K", "Q6_K", "Q6_K"), 1024, 512, 8, 2, True, 0),
    (("Q8_0", "Q8_0", "Q4_0"), 2048, 768, 10, 3, True, 0),
    (("Q5_K", "Q5_K", "Q4_1"), 2048, 512, 8, 2, True, 512),
]


@pytest.mark.parametrize("T", [1, 3])
@pytest.mark.parametrize("types,H,I,E,k,norm,Is", CASES)
def test_decode_general_layer_vs_oracle(types, H, I, E, k, norm, Is, T):
    from larder_amd import layer as lay
    rng = np.random.default_rng(H + I + E + T + len(types[2]))
    L = make_layer(rng, types, H, I, E, k, norm, Is)
    # a Q6_K / Q8_0 down under one Q4 gate/up type stays on the prepared chain (h in the Q4_K / Q4_0 order); the
    # rest go general
    assert lay.prepared_chain(L) == (types[2] in ("Q6_K", "Q8_0") and types[0] == types[1]
                                     and types[0] in ("Q4_0", "Q4_K"))
    if Is and Is % I == 0:
        assert L.folded is not None
    x = dev(rng.standard_normal((T, H)).astype(np.float16))
    B = lay.DecodeBuffers(L, T)
    out = torch.empty((T, H), dtype=torch.float32, device="cuda")
    lay.decode(L, x, B, out, residual=x)
    torch.cuda.synchronize()
    xs = host(x.float())
    lg, ids, want = oracle_out(L, x, residual=xs)
    assert np.array_equal(host(B.logits)[:, :E].view(np.uint32), lg.view(np.uint32))
    assert (host(B.ids).astype(np.uint32) == ids).all()
    if L.folded is not None:  # the shared slices ride as experts E .. E + m - 1 in slots k .. k + m - 1
        assert (host(B.ids_ext)[:, k:] == E + np.arange(L.n_shared)).all()
    assert moe.rel_l2(host(out) - xs, want - xs) < BAR


def test_decode_general_given_logits():
    """No router weight: the top-k over given logits, then the same chain."""
    from larder_amd import layer as lay
    rng = np.random.default_rng(77)
    types, H, I, E, k = ("Q4_K", "Q4_K", "Q6_K"), 2048, 512, 16, 4
    L = make_layer(rng, types, H, I, E, k, True, router=False)
    T = 2
    x = dev(rng.standard_normal((T, H)).astype(np.float16))
    lg = rng.standard_normal((T, E)).astype(np.float32)
    B = lay.DecodeBuffers(L, T)
    out = torch.empty((T, H), dtype=torch.float16, device="cuda")
    lay.decode(L, x, B, out, logits=dev(lg))
    torch.cuda.synchronize()
    ids, _, want = moe.layer(host(x.float()), lg, tuple(host(b) for b in (L.wg, L.wu, L.wd)), types, k, True)
    assert (host(B.ids).astype(np.uint32) == ids).all()
    assert moe.rel_l2(host(out.float()), want) < BAR


def test_decode_general_folded_matches_apart():
    """The 35B mix with its shared expert folded in (slots k .. k + 1) and run apart: equal ids, outputs within the
    bar of each other."""
    from larder_amd import layer as lay
    rng = np.random.default_rng(5)
    L = make_layer(rng, ("Q4_K", "Q4_K", "Q6_K"), 2048, 512, 12, 4, True, Is=1024)
    U = lay.MoELayer(L.wg, L.wu, L.wd, L.types, L.k, L.norm, wr=L.wr, shared=L.shared, wsg=L.wsg,
                     fold_shared=False)
    assert L.n_shared == 2 and U.folded is None
    x = dev(rng.standard_normal((2, 2048)).astype(np.float16))
    outs = []
    for layer in (L, U):
        B = lay.DecodeBuffers(layer, 2)
        out = torch.empty((2, 2048), dtype=torch.float32, device="cuda")
        lay.decode(layer, x, B, out)
        torch.cuda.synchronize()
        outs.append((host(out), host(B.ids).copy()))
    assert (outs[0][1] == outs[1][1]).all()
    assert moe.rel_l2(outs[0][0], outs[1][0]) < BAR


def test_decode_general_stack_graph_matches_eager():
    """Two 35B-mix layers (shared expert folded in) as a DecodeStack: a captured step replays to the eager result
    bit for bit, with eager work and a sync between replays."""
    from larder_amd import layer as lay
    rng = np.random.default_rng(11)
    layers = [make_layer(rng, ("Q4_K", "Q4_K", "Q6_K"), 2048, 512, 12, 4, True, Is=512) for _ in range(2)]
    st = lay.DecodeStack(layers, 1)
    xs = dev(rng.standard_normal((4, 1, 2048)).astype(np.float16))
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
        _ = torch.randn(1000, device="cuda").sum().item()
    # the first layer of the last eager step against the oracle (each layer's own parity is the test above)
    B = lay.DecodeBuffers(layers[0], 1)
    out = torch.empty((1, 2048), dtype=torch.float32, device="cuda")
    lay.decode(layers[0], xs[3], B, out, residual=xs[3])
    torch.cuda.synchronize()
    xr = host(xs[3].float())
    _, ids, want = oracle_out(layers[0], xs[3], residual=xr)
    assert (host(B.ids).astype(np.uint32) == ids).all()
    assert moe.rel_l2(host(out) - xr, want - xr) < BAR
