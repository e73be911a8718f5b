"""Pins of the oracle's router-logit restatement (oracle.moe.router_logits_gemv).

The GPU kernels sum x . w in a fixed order, and the oracle restates that order so that the expert ids can be
checked bit for bit from x and the router weight. These cases are built so that the order decides the result
(2^24 + 1 rounds back to 2^24 in float32, 2^24 + 2 does not), with the expected values derived by hand below;
a restatement that chunks, trees or orders the partials differently gets a different number.
"""
import numpy as np

from oracle import moe

BIG = np.float32(2.0 ** 24)


def _one_hot_products(H, placements):
    """x, w (f16, [1, H] / [1, H]) with product x_i w_i = v at each (i, v) and 0 elsewhere; v in {2^24, 1, 2, 4}."""
    x = np.zeros((1, H), np.float16)
    w = np.zeros((1, H), np.float16)
    for i, v in placements:
        if v == BIG:
            x[0, i], w[0, i] = 2048.0, 8192.0
        else:
            x[0, i], w[0, i] = float(v), 1.0
    return x, w


def test_gemv_order_small_integers_equal_exact_dot():
    rng = np.random.default_rng(0)
    for H in (2048, 4096):
        x = rng.integers(-3, 4, (3, H)).astype(np.float16)
        w = rng.integers(-3, 4, (5, H)).astype(np.float16)
        want = x.astype(np.float64) @ w.astype(np.float64).T
        assert np.array_equal(moe.router_logits_gemv(x, w), want.astype(np.float32))


def test_gemv_order_waves_left_to_right():
    # H 2048: 256 threads of one 8-element item. Wave 0 (threads 0..63, elements 0..511) totals 2^24; waves 1, 2,
    # 3 total 1 each. Left to right: ((2^24 + 1) + 1) + 1 = 2^24 (each +1 lost). A tree over the waves would give
    # (2^24 + 1) + (1 + 1) = 2^24 + 2.
    x, w = _one_hot_products(2048, [(0, BIG), (512, 1), (1024, 1), (1536, 1)])
    assert moe.router_logits_gemv(x, w)[0, 0] == np.float32(2.0 ** 24)
    # wave 0 = 2^24, wave 1 = 2: (2^24 + 2) + 0 + 0 = 2^24 + 2
    x, w = _one_hot_products(2048, [(0, BIG), (512, 2)])
    assert moe.router_logits_gemv(x, w)[0, 0] == np.float32(2.0 ** 24 + 2)


def test_gemv_order_items_of_a_thread():
    # H 4096: thread 0 holds items 0 and 256 (elements 0..7, then 2048..2055), summed in that order from zero:
    # 2^24 + 1 + 1 -> 2^24; thread 1 (elements 8..15) holds 2 -> wave tree (2^24 + 2) = 2^24 + 2.
    x, w = _one_hot_products(4096, [(0, BIG), (2048, 1), (2049, 1), (8, 2)])
    assert moe.router_logits_gemv(x, w)[0, 0] == np.float32(2.0 ** 24 + 2)
    # inside a wave the tree pairs neighbours: threads 0 (2^24) and 1 (1) -> 2^24, thread 2 (1) + thread 3 (0) = 1,
    # then 2^24 + 1 -> 2^24
    x, w = _one_hot_products(2048, [(0, BIG), (8, 1), (16, 1)])
    assert moe.router_logits_gemv(x, w)[0, 0] == np.float32(2.0 ** 24)


def test_planted_order_mistake_is_caught():
    """A restatement that sums an item's 8 products as a tree instead of a chain from zero keeps the ones that the
    chain loses (2^24 + 1 rounds back to 2^24, ties to even): the pins above and below would catch that mistake."""
    x, w = _one_hot_products(2048, [(0, BIG)] + [(i, 1) for i in range(1, 8)])
    assert moe.router_logits_gemv(x, w)[0, 0] == BIG
    p = (x.astype(np.float32) * w.astype(np.float32))[0, :8]
    assert moe._tree(p) == np.float32(2.0 ** 24 + 6) != moe.router_logits_gemv(x, w)[0, 0]
    # the ones of item 1 (elements 8..15) stay in their own chain (8), then meet 2^24 in the wave tree: 2^24 + 8
    x, w = _one_hot_products(2048, [(0, BIG)] + [(i, 1) for i in range(8, 16)])
    assert moe.router_logits_gemv(x, w)[0, 0] == np.float32(2.0 ** 24 + 8)


def _gemv_order_loops(x, w):
    """k_router_gemv's order written out thread by thread (256 threads, items i, i + 256, ..., 8 products a step,
    wave trees, waves left to right), for tiny shapes only: the chunked, vectorised oracle must give its bits."""
    x = np.asarray(x, np.float32)
    H = x.shape[-1]
    w = np.asarray(w, np.float32).reshape(-1, H)
    nit = H // 8
    out = np.zeros((x.shape[0], w.shape[0]), np.float32)
    for t in range(x.shape[0]):
        for r in range(w.shape[0]):
            chains = np.zeros(256, np.float32)
            for th in range(256):
                a = np.float32(0)
                for it in range(th, nit, 256):
                    for e in range(8):
                        a = np.float32(a + np.float32(x[t, 8 * it + e] * w[r, 8 * it + e]))
                chains[th] = a
            wv = []
            for q in range(4):
                v = chains[64 * q:64 * q + 64]
                while v.size > 1:
                    v = (v[0::2] + v[1::2]).astype(np.float32)
                wv.append(v[0])
            out[t, r] = np.float32(np.float32(np.float32(wv[0] + wv[1]) + wv[2]) + wv[3])
    return out


def test_gemv_order_vectorised_equals_thread_loops():
    """The chunked oracle against the thread-by-thread loops on random f16 / bf16 rows whose sums round differently
    in different orders (values spanning 2^-8 .. 2^8), at hidden sizes with one, two and a partial second item a
    thread."""
    import torch
    rng = np.random.default_rng(7)
    for H in (2048, 2560, 4096):
        x = (rng.standard_normal((2, H)) * np.exp2(rng.integers(-8, 9, (2, H)))).astype(np.float16)
        w = torch.from_numpy(rng.standard_normal((3, H)).astype(np.float32) * 0.02).bfloat16().float().numpy()
        got = moe.router_logits_gemv(x, w)
        want = _gemv_order_loops(x, w)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), H
