"""GPU parity of the fused decode stack (lmoe_stack_decode: every layer of a batch-1 step in one launch) against the
CPU oracle, layer by layer, from each layer's own input x_l:
  * router logits bit-exact against oracle.moe.router_logits_stack (the kernel's fixed reduction order);
  * expert ids bit-exact (ties to the lowest index), scores within 2e-6;
  * the layer's MoE output within 2e-3 relative L2 of the fp32 dequant-then-matmul;
  * x_{l+1} = f16(x_l + y_l) bit for bit (the residual hand-off between layers);
plus repeated launches on one workspace (the epoch) giving identical bits."""
import numpy as np
import pytest
import torch

from oracle import moe

pytestmark = pytest.mark.gpu

BAR = 2e-3


def host(t):
    return t.detach().cpu().numpy()


def _stack(cfg, L, seed, **kw):
    from larder_amd import stack, workloads
    g = torch.Generator(device="cuda").manual_seed(seed)
    layers = [workloads.make_layer(cfg, g) for _ in range(L)]
    return layers, stack.Stack(layers, trace=True, **kw)


def _picked(buf, ids):
    """The picked experts' blocks on the host, and slots remapped to them."""
    return host(buf[torch.as_tensor(ids.astype(np.int64), device=buf.device)])


def _check_layers(layers, st, x, out, cfg):
    print(f"stack check: L {st.L} H {st.H} E {st.E} k {st.k} I {st.I} Is {st.Is}", flush=True)
    xs = host(st.layer_inputs())                    # [L, H] f16
    lg = host(st.logits())                          # [L, E (+1)]
    ids_gpu, sc_gpu, y_gpu = host(st.ids).astype(np.uint32), host(st.scores), host(st.y)
    E, k = st.E, st.k
    for l, Ly in enumerate(layers):
        x_l = xs[l:l + 1]
        want_lg = moe.router_logits_stack(x_l, host(Ly.wr))
        assert np.array_equal(lg[l:l + 1, :E].view(np.uint32), want_lg.view(np.uint32)), f"layer {l} logits"
        if st.Is:
            want_g = moe.router_logits_stack(x_l, host(Ly.wsg).reshape(1, -1))
            assert np.array_equal(lg[l, E:E + 1].view(np.uint32), want_g[0].view(np.uint32)), f"layer {l} gate"
        ids, sc = moe.router(want_lg, k, cfg["norm"])
        assert np.array_equal(ids_gpu[l], ids[0]), f"layer {l} ids {ids_gpu[l]} vs {ids[0]}"
        assert np.allclose(sc_gpu[l], sc[0], rtol=2e-6, atol=1e-7), f"layer {l} scores"
        w = tuple(_picked(b, ids[0]) for b in (Ly.wg, Ly.wu, Ly.wd))
        shared = tuple(host(b[0]) for b in Ly.shared) if Ly.shared is not None else None
        _, y = moe.gemv(x_l.astype(np.float32), w, np.arange(k), k, cfg["types"])
        gate = sh = None
        if shared is not None:
            sh = moe.shared_expert(x_l.astype(np.float32), *shared, cfg["types"])
            gate = want_g[:, 0]
        want_y = moe.combine(y.reshape(1, k, -1), sc, sh, gate)
        err = moe.rel_l2(y_gpu[l], want_y[0])
        assert err < BAR, f"layer {l}: rel L2 {err:.3g}"
        nxt = (x_l.astype(np.float32) + y_gpu[l:l + 1]).astype(np.float16)
        have = xs[l + 1:l + 2] if l + 1 < st.L else host(out).reshape(1, -1)
        assert np.array_equal(nxt.view(np.uint16), have.view(np.uint16)), f"layer {l} residual hand-off"


@pytest.mark.parametrize("L", [1, 3])
def test_stack_cfg2_shape(L):
    from larder_amd import workloads
    cfg = workloads.CONFIGS[2]
    layers, st = _stack(cfg, L, 10 + L)
    g = torch.Generator(device="cuda").manual_seed(L)
    x = torch.randn((cfg["H"],), generator=g, device="cuda").half()
    out = torch.empty_like(x)
    st.step(x, out)
    st.check()
    _check_layers(layers, st, x, out, cfg)


def test_stack_cfg1_shape_shared_expert():
    """E 60, top-4 without renormalisation, I 1408, a 5632-wide shared expert with a sigmoid gate."""
    from larder_amd import workloads
    cfg = workloads.CONFIGS[1]
    layers, st = _stack(cfg, 2, 21)
    x = torch.randn((cfg["H"],), generator=torch.Generator(device="cuda").manual_seed(3), device="cuda").half()
    out = torch.empty_like(x)
    st.step(x, out)
    st.check()
    _check_layers(layers, st, x, out, cfg)


def test_stack_cfg5_shape_q4_k():
    """H 4096, E 512, top-10, I 512, shared expert 512, Q4_K blocks."""
    from larder_amd import workloads
    cfg = workloads.CONFIGS[5]
    layers, st = _stack(cfg, 2, 31)
    x = torch.randn((cfg["H"],), generator=torch.Generator(device="cuda").manual_seed(4), device="cuda").half()
    out = torch.empty_like(x)
    st.step(x, out)
    st.check()
    _check_layers(layers, st, x, out, cfg)


def test_stack_ties_to_lowest_index():
    """Router rows planted equal: equal logits are picked lowest index first, across the k-th place too."""
    from larder_amd import workloads
    cfg = dict(workloads.CONFIGS[2], E=64)
    layers, st = _stack(cfg, 2, 41)
    for Ly in layers:
        # experts 3, 17, 40 and 63 share a large row: they tie at the top; 5, 9, 50 share a smaller one
        Ly.wr[[3, 17, 40, 63]] = Ly.wr[3] * 4
        Ly.wr[[5, 9, 50]] = Ly.wr[5] * 3
    x = torch.randn((cfg["H"],), generator=torch.Generator(device="cuda").manual_seed(5), device="cuda").half()
    out = torch.empty_like(x)
    st.step(x, out)
    st.check()
    _check_layers(layers, st, x, out, cfg)


def test_stack_repeated_launches_same_bits():
    """Five launches on one workspace (five epochs) from the same input give the same output bits, and a fresh
    input in between is honoured (no stale hand-off word is taken)."""
    from larder_amd import workloads
    cfg = dict(workloads.CONFIGS[2], E=32)
    layers, st = _stack(cfg, 4, 51)
    g = torch.Generator(device="cuda").manual_seed(6)
    xa = torch.randn((cfg["H"],), generator=g, device="cuda").half()
    xb = torch.randn((cfg["H"],), generator=g, device="cuda").half()
    outs = []
    for i in range(5):
        o = torch.empty_like(xa)
        st.step(xa if i % 2 == 0 else xb, o)
        outs.append(o)
    st.check()
    assert torch.equal(outs[0], outs[2]) and torch.equal(outs[0], outs[4])
    assert torch.equal(outs[1], outs[3])
    assert not torch.equal(outs[0], outs[1])
    _check_layers(layers, st, xa, outs[4], cfg)
