"""The stream layout of Q4 expert matrices (lmoe_stream_repack) and the grouped GEMMs that read it
(lmoe_grouped_gate_up_sl / lmoe_grouped_down_sl):
  * the repack against an independent numpy restatement of the permutation, byte for byte (Q4_0 and Q4_K);
  * the GEMMs on stream copies bit-equal to the GGUF-layout GEMMs (h and y), over every tile height the Q4_0 kernel
    takes (32 with split-K, 64, 128) and Q4_K's 64, on ragged groupings with empty experts and short groups;
  * a prefill layer with MoELayer.keep_stream() bit-equal to the same layer without it, and within the bar of the
    oracle."""
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


def stream_order(w, t):
    """The stream layout by numpy indexing: w uint8 [E, rows, row bytes] -> flat uint8."""
    E, rows, rb = w.shape
    q = np.arange(256)
    feat = 16 * (q >> 5) + (q & 15)
    half = (q >> 4) & 1
    out = []
    for e in range(E):
        for fb in range(rows // 128):
            f0 = fb * 128
            if t == "Q4_0":
                for kk in range(rb // 36):
                    heads = np.stack([w[e, f0 + f, 36 * kk + 16 * h: 36 * kk + 16 * h + 16] for f, h in zip(feat, half)])
                    tails = w[e, f0:f0 + 128, 36 * kk + 32: 36 * kk + 36]
                    out += [heads.reshape(-1), tails.reshape(-1)]
            else:
                for sb in range(rb // 144):
                    out.append(w[e, f0:f0 + 128, 144 * sb: 144 * sb + 16].reshape(-1))
                    for pr in range(4):
                        o = 144 * sb + 16 + 32 * pr
                        out.append(np.stack([w[e, f0 + f, o + 16 * h: o + 16 * h + 16]
                                             for f, h in zip(feat, half)]).reshape(-1))
    return np.concatenate(out)


@pytest.mark.parametrize("t,rows,cols", [("Q4_0", 256, 512), ("Q4_0", 384, 128), ("Q4_K", 256, 512),
                                         ("Q4_K", 128, 1024)])
def test_repack_is_the_permutation(t, rows, cols):
    from larder_amd import _lib, grouped
    rng = np.random.default_rng(rows + cols)
    w = gguf.random_experts(rng, 3, rows, cols, t)
    assert _lib.lib().lmoe_stream_bytes(_lib.qcode(t), 3, rows, cols) == w.nbytes
    got = host(grouped.stream_copy(dev(w), t)).reshape(-1)
    assert np.array_equal(got, stream_order(w, t))


def _ragged(rng, R, E):
    s = rng.integers(2, E, R)
    s[: R // 3] = 0                      # one expert over several tiles
    s[R // 3: R // 3 + 5] = E - 1        # a short group
    return s[rng.permutation(R)].astype(np.int32)   # expert 1 empty


@pytest.mark.parametrize("t,bm,ks", [("Q4_0", 32, 1), ("Q4_0", 32, 2), ("Q4_0", 64, 1), ("Q4_0", 128, 1),
                                     ("Q4_K", 64, 1)])
def test_stream_gemms_bit_equal(t, bm, ks):
    from larder_amd import grouped
    H, I, E = (2048, 768, 6) if t == "Q4_0" else (1024, 512, 6)
    rng = np.random.default_rng(bm * 7 + ks)
    wg, wu, wd = (dev(gguf.random_experts(rng, E, r, c, t)) for r, c in ((I, H), (I, H), (H, I)))
    sg, su, sd = (grouped.stream_copy(w, t) for w in (wg, wu, wd))
    R = 300
    ids = _ragged(rng, R, E)
    G = grouped.Grouping(R, E, bm=bm).run(dev(ids))
    x = dev(rng.standard_normal((R, H)).astype(np.float32)).half()
    types = (t,) * 3
    outs = []
    for sl in (None, (sg, su, sd)):
        h = torch.empty((R, I), dtype=torch.float16, device="cuda")
        grouped.gate_up(x, G, 1, wg, wu, types, h, ksplit=ks, sl=sl[:2] if sl else None)
        y = torch.empty((R, H), dtype=torch.float32, device="cuda")
        grouped.down(h, G, wd, t, y, ksplit=ks, sl=sl[2] if sl else None)
        torch.cuda.synchronize()
        outs.append((host(h).view(np.uint16), host(y).view(np.uint32)))
    n = int(host(G.offsets)[-1])
    assert np.array_equal(outs[0][0][:n], outs[1][0][:n])
    assert np.array_equal(outs[0][1][:n], outs[1][1][:n])


@pytest.mark.parametrize("cfgid,T", [(4, 64), (5, 300), (1, 40)])
def test_prefill_with_stream_copies(cfgid, T, monkeypatch):
    """cfg4 (Q4_0, 32-row tiles), cfg5's Q4_K layer (64 experts, no shared expert) and cfg1 (Q4_0 with its 5,632-wide
    shared expert, router logits from the router weight): bit-equal with and without the copies at one K split
    (on stream copies the path takes no split-K, where the GGUF layout's rule splits cfg4's tiles), and within the
    bar of the oracle either way."""
    from larder_amd import grouped, workloads
    monkeypatch.setenv("LMOE_KSPLIT", "1")
    cfg = dict(workloads.CONFIGS[cfgid])
    if cfgid == 5:
        cfg.update(E=64, Is=0)          # the Q4_K layer at cfg5's shapes, fewer experts
    g = torch.Generator(device="cuda").manual_seed(cfgid)
    L = workloads.make_layer(cfg, g)
    lg = workloads.skewed_logits(T, cfg["E"], g) if cfgid != 1 else None
    x = torch.randn((T, cfg["H"]), generator=g, device="cuda").half()
    B = grouped.PrefillBuffers(L, T)
    plain = torch.empty((T, cfg["H"]), dtype=torch.float32, device="cuda")
    grouped.prefill(L, x, B, plain, logits=lg)
    held = L.keep_stream()
    want_held = sum(w.numel() for w in (L.wg, L.wu, L.wd)) + (sum(w.numel() for w in L.shared) if L.shared else 0)
    assert held == want_held
    out = torch.empty_like(plain)
    grouped.prefill(L, x, B, out, logits=lg)
    torch.cuda.synchronize()
    assert torch.equal(out, plain)
    w = tuple(host(b) for b in (L.wg, L.wu, L.wd))
    if cfgid == 1:
        lg_h = moe.router_logits_gemv(host(x.float()), host(L.wr.float()))  # routing pinned from x
        _, _, want = moe.layer(host(x.float()), lg_h, w, cfg["types"], cfg["k"], cfg["norm"],
                               shared=tuple(host(b[0]) for b in L.shared), shared_gate_w=host(L.wsg.float()))
    else:
        _, _, want = moe.layer(host(x.float()), host(lg), w, cfg["types"], cfg["k"], cfg["norm"])
    assert moe.rel_l2(host(out), want) < BAR
