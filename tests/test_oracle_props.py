"""The oracle pinned where the reference holds no vectors: closed forms, known answers, brute force on small
inputs, library routines, invariants, and planted mistakes that those checks must catch."""
import numpy as np
import pytest

from oracle import gguf, moe


# ---- Q4_0 quantizer: ggml's quantize_row_q4_0_ref rule on blocks whose answers are exact in binary ----------------

def test_q4_0_known_answer_exact_steps():
    # x = (j - 8) / 4 twice: the first largest magnitude is -2 -> d = 0.25, id = 4, q = trunc(j - 8 + 8.5) = j
    j = np.arange(16, dtype=np.float32)
    x = np.concatenate([(j - 8) / 4, (j - 8) / 4]).astype(np.float32)
    b = gguf.quantize_q4_0(x[None])[0]
    assert b[0:2].view(np.float16)[0] == np.float16(0.25)
    assert (b[2:18] == (j.astype(np.uint8) | (j.astype(np.uint8) << 4))).all()
    assert (gguf.dequant(b, "Q4_0") == x).all()


def test_q4_0_known_answer_clamp_and_zero():
    x = np.zeros(32, np.float32)
    x[3], x[20] = 2.0, -2.0          # largest magnitude first seen positive: d = -0.25, id = -4
    b = gguf.quantize_q4_0(x[None])[0]
    assert b[0:2].view(np.float16)[0] == np.float16(-0.25)
    w = gguf.dequant(b, "Q4_0")
    assert w[3] == 2.0               # q = trunc(-8 + 8.5) = 0 -> (0 - 8) * -0.25
    assert w[20] == -1.75            # q = trunc(8 + 8.5) = 16, clamped to 15 -> 7 * -0.25
    assert (np.delete(w, [3, 20]) == 0).all()
    z = gguf.quantize_q4_0(np.zeros((1, 32), np.float32))[0]
    # d = 0.0 / -8 = -0.0 (f16 0x8000), id = 0, every q = trunc(8.5) = 8
    assert z[0:2].view(np.uint16)[0] == 0x8000 and (z[2:] == 0x88).all()


def test_q4_0_round_trip_bound():
    rng = np.random.default_rng(1)
    w = rng.standard_normal((64, 256)).astype(np.float32) * 0.02
    q = gguf.quantize_q4_0(w)
    back = gguf.dequant_matrix(q, "Q4_0")
    d = np.abs(q.reshape(-1, 18)[:, 0:2].copy().view(np.float16)[:, 0].astype(np.float32))
    err = np.abs(back - w).reshape(-1, 32)
    # half a step, or a whole step where the clamp at 15 bites, plus the f16 rounding of d over 8 steps
    assert (err <= d[:, None] * 1.0 + 8 * np.abs(d[:, None]) * 2 ** -10 + 1e-9).all()
    assert np.sqrt(np.mean((back - w) ** 2)) < 0.02 * 0.12


def test_q4_k_round_trip_and_validity():
    rng = np.random.default_rng(2)
    w = rng.standard_normal((16, 512)).astype(np.float32) * 0.02
    q = gguf.quantize_q4_k(w)
    assert q.shape == (16, 2 * 144) and gguf.valid(q, "Q4_K")
    back = gguf.dequant_matrix(q, "Q4_K")
    assert np.sqrt(np.mean((back - w) ** 2)) < 0.02 * 0.15
    # the 6-bit scale/min packing round-trips through get_scale_min_k4 for every value 0..63
    sc = np.arange(64, dtype=np.uint8)
    for off in range(8):
        v = np.roll(sc, off)[:8]
        m = np.roll(sc, 3 * off + 1)[:8]
        s = np.zeros((1, 12), np.uint8)
        s[0, 0:4] = (v[0:4] & 63) | ((v[4:8] >> 4) << 6)
        s[0, 4:8] = (m[0:4] & 63) | ((m[4:8] >> 4) << 6)
        s[0, 8:12] = (v[4:8] & 0xF) | ((m[4:8] & 0xF) << 4)
        gs, gm = gguf.scale_min_k4(s)
        assert (gs[0] == v).all() and (gm[0] == m).all()


def test_q4_k_single_sub_block_closed_form():
    # one super-block, only sub-block 5 non-zero: y = d * sc * q - dmin * m there, -dmin * m_j elsewhere
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([0.5], np.float16).view(np.uint8)
    b[2:4] = np.array([0.25], np.float16).view(np.uint8)
    sc = np.array([0, 0, 0, 0, 0, 37, 0, 0], np.uint8)
    m = np.array([1, 2, 3, 4, 5, 6, 7, 63], np.uint8)
    b[4:8] = (sc[0:4] & 63) | ((sc[4:8] >> 4) << 6)
    b[8:12] = (m[0:4] & 63) | ((m[4:8] >> 4) << 6)
    b[12:16] = (sc[4:8] & 0xF) | ((m[4:8] & 0xF) << 4)
    q = np.arange(32) % 16
    b[16 + 64:16 + 96] = q.astype(np.uint8) << 4      # sub-block 5 = high nibbles of qs[64:96] (c = 2)
    y = gguf.dequant(b, "Q4_K").reshape(8, 32)
    assert (y[5] == np.float32(0.5 * 37) * q.astype(np.float32) - np.float32(0.25 * 6)).all()
    for j in (0, 1, 2, 3, 4, 6, 7):
        assert (y[j] == -np.float32(0.25) * np.float32(m[j])).all()


# ---- router ------------------------------------------------------------------------------------------------------

def _brute_topk(row, k):
    pairs = sorted(((-float(v), i) for i, v in enumerate(row)))
    return [i for _, i in pairs[:k]]


@pytest.mark.parametrize("E,k", [(60, 4), (128, 8), (512, 10), (7, 7)])
def test_topk_matches_brute_force_with_ties(E, k):
    rng = np.random.default_rng(E + k)
    for r in range(40):
        row = rng.standard_normal(E).astype(np.float32)
        if r % 5 == 0:
            j = rng.integers(0, E, 6)
            row[j] = row[j[0]]
        if r % 7 == 0:
            row = np.round(row * 2) / 2
        if r % 11 == 0:
            row[:] = 0.5                      # all tied: the lowest k indices
        got = moe.topk_ids(row, k).tolist()
        assert got == _brute_topk(row, k)


def test_router_scores_and_renorm():
    rng = np.random.default_rng(3)
    lg = rng.standard_normal((32, 128)).astype(np.float32) * 2
    g = moe.softmax(lg)
    assert np.allclose(g.sum(-1), 1, atol=1e-6)
    ids, s = moe.router(lg, 8, False)
    e = np.exp(lg.astype(np.float64) - lg.max(-1, keepdims=True))
    want = np.take_along_axis(e / e.sum(-1, keepdims=True), ids.astype(np.int64), -1)
    assert np.allclose(s, want, rtol=1e-6)
    ids2, s2 = moe.router(lg, 8, True)
    assert (ids2 == ids).all() and np.allclose(s2.sum(-1), 1, atol=1e-6)
    assert np.allclose(s2, want / want.sum(-1, keepdims=True), rtol=1e-6)


# ---- grouping ----------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("R,E", [(0, 4), (1, 4), (100, 8), (4096, 128), (5000, 60)])
def test_group_rows_is_the_stable_sort(R, E):
    rng = np.random.default_rng(R + E)
    ids = rng.integers(0, E + 3, R).astype(np.uint32)        # a few ids past the last expert
    counts, offsets, order, inv = moe.group_rows(ids, E)
    key = np.where(ids < E, ids, E)
    assert (order == np.argsort(key, kind="stable")).all()
    assert (np.sort(order) == np.arange(R)).all() and (order[inv] == np.arange(R)).all()
    assert (counts == np.bincount(key, minlength=E + 1)[:E]).all()
    assert offsets[0] == 0 and (np.diff(offsets.astype(np.int64)) == counts).all()
    for e in range(E):
        seg = order[offsets[e]:offsets[e + 1]]
        assert (ids[seg] == e).all() and (np.diff(seg.astype(np.int64)) > 0).all()
    assert (ids[order[offsets[E]:]] >= E).all()


# ---- the layer -------------------------------------------------------------------------------------------------

def test_layer_closed_form_float64():
    """Each token's output equals sum_j s_j Wd_e (silu(Wg_e x) * (Wu_e x)) done in float64 directly."""
    rng = np.random.default_rng(4)
    H, I, E, k, T = 128, 64, 6, 3, 5
    w = tuple(gguf.random_experts(rng, E, r, c, "Q4_0") for r, c in ((I, H), (I, H), (H, I)))
    x = rng.standard_normal((T, H)).astype(np.float16)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    ids, s, out = moe.layer(x, lg, w, ("Q4_0",) * 3, k, True)
    wg, wu, wd = (gguf.dequant_matrix(b, "Q4_0").astype(np.float64) for b in w)
    for t in range(T):
        acc = np.zeros(H)
        for j in range(k):
            e = int(ids[t, j])
            xt = x[t].astype(np.float64)
            g, u = wg[e] @ xt, wu[e] @ xt
            acc += float(s[t, j]) * (wd[e] @ (g / (1 + np.exp(-g)) * u))
        assert moe.rel_l2(out[t], acc) < 1e-5


def test_layer_shared_expert_and_residual():
    rng = np.random.default_rng(5)
    H, I, Is, E, k, T = 64, 64, 128, 4, 2, 3
    w = tuple(gguf.random_experts(rng, E, r, c, "Q4_0") for r, c in ((I, H), (I, H), (H, I)))
    sh = tuple(gguf.random_experts(rng, 1, r, c, "Q4_0")[0] for r, c in ((Is, H), (Is, H), (H, Is)))
    wsg = rng.standard_normal(H).astype(np.float32) * 0.02
    x = rng.standard_normal((T, H)).astype(np.float32)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    res = rng.standard_normal((T, H)).astype(np.float32)
    _, _, base = moe.layer(x, lg, w, ("Q4_0",) * 3, k, False)
    _, _, full = moe.layer(x, lg, w, ("Q4_0",) * 3, k, False, shared=sh, shared_gate_w=wsg, residual=res)
    sg, su, sd = (gguf.dequant_matrix(b, "Q4_0").astype(np.float64) for b in sh)
    x64 = x.astype(np.float64)
    g, u = x64 @ sg.T, x64 @ su.T
    shared = (g / (1 + np.exp(-g)) * u) @ sd.T
    gate = 1 / (1 + np.exp(-(x64 @ wsg.astype(np.float64))))
    assert moe.rel_l2(full, base + gate[:, None] * shared + res) < 1e-5


def test_gemv_slot_row_mapping():
    """gemv's slot s reads x row s // topk (gguf_experts.py:600-607): permuting x rows permutes outputs."""
    rng = np.random.default_rng(6)
    H, I, E = 64, 64, 5
    w = tuple(gguf.random_experts(rng, E, r, c, "Q4_0") for r, c in ((I, H), (I, H), (H, I)))
    x = rng.standard_normal((3, H)).astype(np.float32)
    slots = np.array([0, 4, 1, 1, 2, 3])
    _, y = moe.gemv(x, w, slots, 2, ("Q4_0",) * 3)
    _, y1 = moe.gemv(x[[2, 0, 1]], w, slots[[4, 5, 0, 1, 2, 3]], 2, ("Q4_0",) * 3)
    assert np.allclose(y[[4, 5, 0, 1, 2, 3]], y1)
    _, bad = moe.gemv(x, w, np.array([0, 7]), 1, ("Q4_0",) * 3)
    assert (bad[1] == 0).all()


# ---- planted mistakes: each check above must catch a plausible slip in the oracle ----------------------------------

def test_planted_nibble_order_mistake_is_caught(monkeypatch):
    from pathlib import Path
    z = np.load(Path(__file__).resolve().parent / "golden" / "dequant_q4.npz")

    def wrong(b):   # weights 2j, 2j+1 from byte j instead of j, j + 16
        qs = b[:, 2:18]
        q = np.stack([qs & 0xF, qs >> 4], axis=2).reshape(-1, 32).astype(np.int32)
        return (q - 8).astype(np.float32) * gguf._f16(b, 0)[:, None]

    monkeypatch.setitem(gguf._DQ, "Q4_0", wrong)
    got = gguf.dequant(z["Q4_0_blocks"].reshape(-1), "Q4_0")
    assert not (got.view(np.uint32) == z["Q4_0_want"].view(np.uint32)).all()


def test_planted_scale_packing_mistake_is_caught(monkeypatch):
    from pathlib import Path
    z = np.load(Path(__file__).resolve().parent / "golden" / "dequant_q4.npz")

    def wrong(s):   # high bits of sub-blocks 4..7 taken from the m bytes instead of the sc bytes
        s = s.astype(np.uint8)
        sc = np.concatenate([s[:, 0:4] & 63, (s[:, 8:12] & 0xF) | ((s[:, 4:8] >> 6) << 4)], axis=1)
        m = np.concatenate([s[:, 4:8] & 63, (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)], axis=1)
        return sc.astype(np.float32), m.astype(np.float32)

    monkeypatch.setattr(gguf, "scale_min_k4", wrong)
    got = gguf.dequant(z["Q4_K_blocks"].reshape(-1), "Q4_K")
    assert not (got.view(np.uint32) == z["Q4_K_want"].view(np.uint32)).all()


def test_planted_tie_mistake_is_caught():
    row = np.array([1.0, 3.0, 3.0, 0.0, 3.0], np.float32)
    largest_first = list(np.argsort(row, kind="stable")[::-1][:2])     # MLX's tie order: larger index first
    assert moe.topk_ids(row, 2).tolist() == [1, 2] == _brute_topk(row, 2)
    assert largest_first != _brute_topk(row, 2)
