"""Router partials: each decode layer's router GEMV folded into its neighbours (the previous layer's down writes the
next router's item partials, gate/up sums them in the router's tree). The ids, scores and prepared h must equal the
three-launch chain's bit for bit, the partials must equal the oracle's item chains, and a stack driven this way must
give the three-launch stack's output bit for bit, eager and as a replayed graph."""
import numpy as np
import pytest
import torch

from oracle import moe

pytestmark = pytest.mark.gpu


def host(t):
    return t.detach().cpu().numpy()


def _cfg(name):
    from larder_amd import workloads
    if name == "cfg2":
        return dict(workloads.CONFIGS[2])
    if name == "cfg2_e16_q4k":      # Q4_K at hidden 2048, 16 experts
        return dict(workloads.CONFIGS[2], E=16, types=("Q4_K",) * 3)
    if name == "cfg1_shared1":      # cfg1's experts with a routed-width shared expert (one folded slice, gate row E)
        return dict(workloads.CONFIGS[1], Is=workloads.CONFIGS[1]["I"])
    if name == "e256":              # the most router rows partials take
        return dict(workloads.CONFIGS[2], E=256, k=4)
    raise KeyError(name)


def _layer(name, seed):
    from larder_amd import workloads
    g = torch.Generator(device="cuda").manual_seed(seed)
    return workloads.make_layer(_cfg(name), g), g


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("name,T", [("cfg2", 1), ("cfg2", 3), ("cfg1_shared1", 2), ("e256", 1)])
def test_router_part_is_the_oracle_item_chain(name, T, xdt):
    from larder_amd import _lib
    L, g = _layer(name, 11)
    x = torch.randn((T, L.H), generator=g, device="cuda").to(xdt)
    wr = L.wr.to(xdt) if xdt != L.wr.dtype else L.wr
    wsg = L.wsg.to(xdt) if L.wsg is not None else None
    rows = L.E + (1 if wsg is not None else 0)
    part = torch.empty((T, L.H // 8, rows), dtype=torch.float32, device="cuda")
    _lib.call("lmoe_router_part", _lib.ptr(x), _lib.dcode(xdt), _lib.ptr(wr), _lib.ptr(wsg), _lib.dcode(xdt), T, L.H,
              L.E, _lib.ptr(part), _lib.stream())
    torch.cuda.synchronize()
    w = host(wr.float()) if wsg is None else np.concatenate([host(wr.float()), host(wsg.float())[None]])
    want = moe.router_partials(host(x.float()), w)
    assert np.array_equal(host(part).view(np.uint32), want.view(np.uint32))
    # and their tree is the router GEMV's logits, bit for bit
    lg = torch.empty((T, rows), dtype=torch.float32, device="cuda")
    xp = torch.empty((T, L.H // 64 * 36), dtype=torch.int32, device="cuda")
    _lib.call("lmoe_router_gemv", _lib.ptr(x), _lib.dcode(xdt), _lib.ptr(wr), _lib.ptr(wsg), _lib.dcode(xdt), T, L.H,
              L.E, _lib.ptr(lg), _lib.ptr(xp), _lib.qcode(L.types[0]), _lib.stream())
    torch.cuda.synchronize()
    assert np.array_equal(host(lg).view(np.uint32), moe.router_logits_from_partials(want).view(np.uint32))


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("name,T", [("cfg2", 1), ("cfg2", 4), ("cfg2_e16_q4k", 2), ("cfg1_shared1", 3), ("e256", 2)])
def test_gate_up_part_equals_the_chain(name, T, xdt):
    """lmoe_router_part + lmoe_moe_gate_up_part against lmoe_router_gemv + lmoe_moe_gate_up_ext: ids, scores and the
    prepared h rows, bit for bit."""
    from larder_amd import _lib, layer as lay
    L, g = _layer(name, 12)
    x = torch.randn((T, L.H), generator=g, device="cuda").to(xdt)
    tg, tu, td = (_lib.qcode(t) for t in L.types)
    (wg, wu, _), m = (L.folded, L.n_shared) if L.folded is not None else ((L.wg, L.wu, L.wd), 0)
    B = lay.DecodeBuffers(L, T)
    rows = L.E + (1 if L.wsg is not None else 0)
    st = _lib.stream()
    _lib.call("lmoe_router_gemv", _lib.ptr(x), _lib.dcode(xdt), _lib.ptr(L.wr), _lib.ptr(L.wsg),
              _lib.dcode(L.wr.dtype), T, L.H, L.E, _lib.ptr(B.logits), _lib.ptr(B.xprep), tg, st)
    _lib.call("lmoe_moe_gate_up_ext", _lib.ptr(B.logits), rows, T, L.k, int(L.norm), _lib.ptr(B.xprep),
              _lib.ptr(B.xprep), _lib.ptr(wg), _lib.ptr(wu), tg, tu, L.E, L.H, L.I, _lib.ptr(B.ids_ext),
              _lib.ptr(B.scores_ext), _lib.ptr(B.hprep), td, m, st)
    torch.cuda.synchronize()
    want = [B.ids_ext.clone(), B.scores_ext.clone(), B.hprep.clone()]
    for t in (B.ids_ext, B.scores_ext, B.hprep):
        t.fill_(-1)
    part = torch.empty((T, 256, rows), dtype=torch.float32, device="cuda")
    _lib.call("lmoe_router_part", _lib.ptr(x), _lib.dcode(xdt), _lib.ptr(L.wr), _lib.ptr(L.wsg),
              _lib.dcode(L.wr.dtype), T, L.H, L.E, _lib.ptr(part), st)
    _lib.call("lmoe_moe_gate_up_part", _lib.ptr(part), _lib.ptr(x), _lib.dcode(xdt), T, L.k, int(L.norm),
              _lib.ptr(wg), _lib.ptr(wu), tg, tu, L.E, L.H, L.I, _lib.ptr(B.ids_ext), _lib.ptr(B.scores_ext),
              _lib.ptr(B.hprep), td, m, st)
    torch.cuda.synchronize()
    for name_, got, exp in zip(("ids", "scores"), (B.ids_ext, B.scores_ext), want[:2]):
        assert torch.equal(got.view(torch.int32), exp.view(torch.int32)), name_
    # gate/up writes the f16 pairs of each 36-dword unit (dwords 0..31); the down kernel derives the sums itself
    P = L.I // 64
    assert torch.equal(B.hprep.view(-1, P, 36)[..., :32], want[2].view(-1, P, 36)[..., :32])
    if xdt != torch.float32:  # the picks are the oracle's top-k of its logits from x (exact f16 / bf16 products)
        lg = moe.router_logits_gemv(host(x.float()), host(L.wr.float()))
        assert np.array_equal(host(B.ids_ext)[:, :L.k].astype(np.uint32), moe.topk_ids(lg, L.k))


@pytest.mark.parametrize("name,T,dt", [("cfg2", 1, torch.float16), ("cfg2", 2, torch.bfloat16),
                                       ("cfg2_e16_q4k", 1, torch.float16), ("cfg1_shared1", 2, torch.float16)])
def test_stack_with_partials_equals_three_launch_stack(name, T, dt):
    """Four layers: x_out of the partials chain equals the three-launch chain's, bit for bit, eager and replayed."""
    from larder_amd import layer as lay, workloads
    cfg = _cfg(name)
    g = torch.Generator(device="cuda").manual_seed(13)
    layers = [workloads.make_layer(cfg, g) for _ in range(4)]
    assert all(lay.part_ok(L) for L in layers)
    a = lay.DecodeStack(layers, T, dtype=dt, parts=True)
    b = lay.DecodeStack(layers, T, dtype=dt, parts=False)
    assert a.parts and not b.parts
    xs = torch.randn((3, T, cfg["H"]), generator=g, device="cuda").to(dt)
    eager = []
    for i in range(3):
        a.x_in.copy_(xs[i])
        b.x_in.copy_(xs[i])
        ya, yb = a.step().clone(), b.step().clone()
        assert torch.equal(ya.view(torch.int16), yb.view(torch.int16)), i
        eager.append(ya)
    graph = a.capture()
    for i in range(3):
        a.x_in.copy_(xs[i])
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(a.x_out, eager[i]), i
        _ = torch.randn(1000, device="cuda").sum().item()     # eager work and a sync between replays


def test_stack_refuses_partials_where_they_do_not_fit():
    """cfg1's 4-slice shared expert (8 slots of 22 units) needs the two-wavefront down: no partials there."""
    from larder_amd import layer as lay, workloads
    g = torch.Generator(device="cuda").manual_seed(14)
    L = workloads.make_layer(workloads.CONFIGS[1], g)
    assert not lay.part_ok(L)
    assert not lay.DecodeStack([L], 1).parts
    with pytest.raises(ValueError, match="router partials"):
        lay.DecodeStack([L], 1, parts=True)
