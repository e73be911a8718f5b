"""GPU parity of the block types beyond Q4_0 / Q4_K (Q4_1, Q8_0, Q5_K, Q6_K) against the CPU oracle, through the
C ABI (larder_amd wrappers): dequant bit for bit (natural order, and the grouped GEMMs' f16 K-order operand to
f16 rounding), the decode chain (pure and mixed layers such as the 35B's Q4_K / Q4_K / Q6_K, slots past the
experts giving zero rows), the down + combine epilogue (scores, gated shared expert, residual) and the grouped
path over dequantized experts, each within the north star's 2e-3 relative L2."""
import numpy as np
import pytest
import torch

from oracle import gguf, moe

pytestmark = pytest.mark.gpu

BAR = 2e-3
NEW = ["Q4_1", "Q8_0", "Q5_K", "Q6_K"]


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.detach().cpu().numpy()


def golden_like(rng, t, n):
    """n blocks of random bytes with finite f16 scales, plus blocks from the quantizer."""
    _, be, bb = gguf.TYPES[t]
    b = rng.integers(0, 256, (n, bb), dtype=np.uint8)
    for at in gguf.HALVES[t]:
        b[:, at:at + 2] = (rng.standard_normal((n, 1)) * 0.01).astype(np.float16).view(np.uint8)
    return b


@pytest.mark.parametrize("t", NEW + ["Q4_0", "Q4_K"])
def test_dequant_bit_exact(t):
    from larder_amd import gguf_experts as ge, grouped
    rng = np.random.default_rng(7)
    _, be, bb = gguf.TYPES[t]
    E, rows, cols = 5, 12, 512
    buf = golden_like(rng, t, E * rows * cols // be).reshape(E, rows, cols // be * bb)
    slots = np.array([4, 0, 9, 2], np.int32)             # 9: past the experts, zeros
    got = host(ge.dequant(dev(buf), dev(slots), t, torch.float32))
    want = moe.dequant_experts(buf, t, [4, 0, 2])
    assert (got[[0, 1, 3]].view(np.uint32) == want.view(np.uint32)).all()
    assert (got[2] == 0).all()
    # the grouped operand: every expert, f16, K order
    w16 = host(grouped.gemm_weights(dev(buf), t).float())
    full = moe.dequant_experts(buf, t).astype(np.float16).astype(np.float32)
    perm = host(grouped.kperm_index(cols, "cuda"))
    assert (w16[..., perm] == full).all()


MIXES = [(("Q4_1", "Q4_1", "Q4_1"), 2048, 768), (("Q8_0", "Q8_0", "Q8_0"), 1024, 512),
         (("Q5_K", "Q5_K", "Q5_K"), 2048, 512), (("Q6_K", "Q6_K", "Q6_K"), 1024, 768),
         (("Q4_K", "Q4_K", "Q6_K"), 2048, 768), (("Q4_0", "Q4_0", "Q8_0"), 2048, 768),
         (("Q6_K", "Q6_K", "Q4_K"), 1024, 512)]


@pytest.mark.parametrize("types,H,I", MIXES)
@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
def test_gemv_chain(types, H, I, xdt):
    from larder_amd import gguf_experts as ge
    rng = np.random.default_rng(H + I + len(types[0]))
    E = 6
    w = tuple(gguf.random_experts(rng, E, r, c, t) for (r, c), t in zip(((I, H), (I, H), (H, I)), types))
    topk, rows = 2, 3
    slots = rng.integers(0, E, rows * topk).astype(np.int32)
    slots[-1] = E + 3                                    # no such expert: zero rows
    x = dev(rng.standard_normal((rows, H)).astype(np.float32)).to(xdt)
    h, y = ge._chain(x, tuple(dev(b) for b in w), dev(slots), topk, types, torch.float32)
    # the Q4 gate/up kernels see x as f16, the general ones as float32
    xs = host(x.float().half().float()) if types[0] in ("Q4_0", "Q4_K") else host(x.float())
    hw, yw = moe.gemv(xs, w, slots, topk, types)
    assert (host(h)[-1] == 0).all() and (host(y)[-1] == 0).all()
    assert moe.rel_l2(host(h), hw) < 1e-5
    assert moe.rel_l2(host(y), yw) < BAR
    y16 = ge.gemv(x, tuple(dev(b) for b in w), dev(slots), topk, "/".join(types), torch.float16)
    assert moe.rel_l2(host(y16.float()), yw) < BAR


@pytest.mark.parametrize("k", [4, 8])
@pytest.mark.parametrize("t", NEW)
def test_down_combine_epilogue(t, k):
    """out[t] = sum_j s_j h[t k + j] . wd[ids] + sigmoid(gate) shared + residual on the general kernels: k 4 at I 512
    is 64 (expert, chunk) items a row, the serial form; k 8 is 128, the flattened forms, where Q6_K takes h as f16
    (v_dot2 on (64 + q) pairs), so its reference rounds h to f16 first. Either way only the summation order is
    left, held to 1e-5."""
    from larder_amd import _lib
    from larder_amd._lib import call, ptr, qcode, stream
    rng = np.random.default_rng(31 + k)
    E, I, H, T = 10, 512, 1024, 3
    wd = gguf.random_experts(rng, E, H, I, t)
    h = rng.standard_normal((T * k, I)).astype(np.float32)
    ids = rng.integers(0, E, T * k).astype(np.int32)
    ids[5] = E + 1
    sc = rng.uniform(0.1, 1.0, (T, k)).astype(np.float32)
    shared = rng.standard_normal((T, H)).astype(np.float32)
    gate = rng.standard_normal(T).astype(np.float32)
    res = rng.standard_normal((T, H)).astype(np.float32)
    out = torch.empty((T, H), dtype=torch.float32, device="cuda")
    dh, did, dsc, dsh, dg, dr = (dev(a) for a in (h, ids, sc, shared, gate, res))
    call("lmoe_gemv_down_combine", ptr(dh), ptr(did), ptr(dsc), T, k, ptr(dev(wd)), qcode(t), E, I, H, ptr(dsh),
         ptr(dg), 1, ptr(dr), _lib.F32, ptr(out), _lib.F32, stream())
    W = moe.dequant_experts(wd, t).astype(np.float64)
    hw = h.astype(np.float16).astype(np.float64) if t == "Q6_K" and k * I // 32 > 64 else h.astype(np.float64)
    want = np.zeros((T, H))
    for r in range(T):
        for j in range(k):
            e = ids[r * k + j]
            if e < E:
                want[r] += sc[r, j] * (W[e] @ hw[r * k + j])
        want[r] += shared[r] / (1.0 + np.exp(-float(gate[r]))) + res[r]
    assert moe.rel_l2(host(out), want) < 1e-5


@pytest.mark.parametrize("types,H,I", [(("Q6_K", "Q6_K", "Q6_K"), 1024, 256), (("Q4_1", "Q4_1", "Q8_0"), 2048, 384),
                                       (("Q4_K", "Q4_K", "Q6_K"), 1024, 512), (("Q5_K", "Q5_K", "Q5_K"), 1024, 512),
                                       (("Q4_0", "Q4_K", "Q4_0"), 1024, 256)])
def test_grouped_dense(types, H, I):
    """gguf_experts.dense over f16-dequantized experts (the f16-weight grouped GEMMs), ragged rows: experts with
    no rows, one row, and several m-tiles."""
    from larder_amd import gguf_experts as ge
    rng = np.random.default_rng(H * 3 + I)
    E = 8
    w = tuple(gguf.random_experts(rng, E, r, c, t) for (r, c), t in zip(((I, H), (I, H), (H, I)), types))
    rows = np.concatenate([np.full(300, 3), np.full(1, 5), rng.integers(0, 3, 60), np.full(7, 7)]).astype(np.int32)
    rng.shuffle(rows)
    x = dev(rng.standard_normal((rows.size, H)).astype(np.float32)).half()
    y = ge.dense(x, tuple(dev(b) for b in w), dev(rows), "/".join(types), torch.float32)
    _, yw = moe.gemv(host(x.float()), w, rows, 1, types)
    assert moe.rel_l2(host(y), yw) < BAR
    for e in (3, 5, 7):
        sel = rows == e
        assert moe.rel_l2(host(y)[sel], yw[sel]) < BAR


def test_prefill_with_resident_f16_weights():
    """A Q4_K / Q4_K / Q6_K layer (and an all-Q8_0 one) through grouped.prefill, dequantizing each call and with
    keep_prefill_f16's resident weights: the same kernels on the same f16 weights, so the same bits; and against
    the oracle."""
    from larder_amd import grouped, layer as lay
    rng = np.random.default_rng(41)
    for types, H, I in ((("Q4_K", "Q4_K", "Q6_K"), 1024, 256), (("Q8_0",) * 3, 1024, 256)):
        E, k, T = 8, 2, 96
        w = tuple(gguf.random_experts(rng, E, r, c, t) for (r, c), t in zip(((I, H), (I, H), (H, I)), types))
        L = lay.MoELayer(*(dev(b) for b in w), types, k, True)
        lg = dev(rng.standard_normal((T, E)).astype(np.float32))
        x = dev(rng.standard_normal((T, H)).astype(np.float32)).half()
        outs = []
        for keep in (False, True):
            if keep:
                assert L.keep_prefill_f16() > 0
            B = grouped.PrefillBuffers(L, T)
            out = torch.empty((T, H), dtype=torch.float32, device="cuda")
            grouped.prefill(L, x, B, out, logits=lg)
            torch.cuda.synchronize()
            outs.append(host(out))
        assert (outs[0] == outs[1]).all()
        _, _, want = moe.layer(host(x.float()), host(lg), w, types, k, True)
        assert moe.rel_l2(outs[1], want) < BAR
